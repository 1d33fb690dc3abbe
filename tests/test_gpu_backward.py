"""Decoder backward on the GPU against autograd of the fp64 dense decoder.

The reference's contract (csrc/ram_attn_topk_addr.cu:119-226,
_cuda_autograd.py:4-180): the gradient flows through the selected weights
only (the top-K selection carries none), and the incoming gradient refers to
the positive weights even when the forward stored them negated.
"""
from __future__ import annotations

import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda"

GRAD_CASES = [
    # B, H, U, P, T, K, re_norm, E
    (2, 4, 2, 16, 48, 4, 0.0, 2),
    (1, 2, 2, 32, 33, 8, 0.5, 1),
    (2, 2, 3, 16, 20, 16, 1.0, 2),
    (1, 3, 5, 4, 17, 12, 0.25, 3),
    (1, 2, 2, 64, 9, 8, 0.0, 0),
    (1, 2, 2, 8, 11, 40, 0.75, 1),   # K > 32: the streaming form
]


def _ops():
    import ramnet_ops  # noqa: F401  (registers torch.ops.ramnet_ops.*)
    return torch.ops.ramnet_ops


def _tol(dtype):
    return 1e-5 if dtype == torch.float32 else 2e-2


def _reference(addr, E, pos, K, re_norm, encode, D, idx=None):
    """fp64 autograd of sum(D * val). With ``idx`` the selection is the
    GPU's (the gradient given a selection, whatever the tie order); without,
    the dense decoder selects."""
    a = addr.double().requires_grad_(True)
    if idx is None:
        ridx, val = oracle.dense_topk_addr(a, E, pos, K, re_norm, False, encode, dtype=torch.float64)
        (val * D.double()).sum().backward()
        return ridx, a.grad
    B, H, U, P, T = addr.shape
    A = P ** U
    inactive = torch.isneginf(a.detach()).all(dim=-2).any(dim=-2)  # (B, H, T)
    logits = a.masked_fill(inactive[:, :, None, None, :], 0)
    scores = oracle.content_scores(oracle.log_softmax_digits(logits, torch.float64))  # (B, H, T, A)
    heads = torch.arange(H).view(1, H, 1, 1)
    shift = (heads < E).long() * pos.long().view(B, 1, 1, T)
    content = torch.remainder(idx.long() % A + shift, A)  # (B, H, K, T)
    s = scores.gather(-1, content.permute(0, 1, 3, 2))  # (B, H, T, K)
    if re_norm != 0:
        s = s - re_norm * s.logsumexp(dim=-1, keepdim=True)
    val = s.exp().masked_fill(inactive[..., None], 0).permute(0, 1, 3, 2)
    (val * D.double()).sum().backward()
    return idx, a.grad


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("neg", [False, True])
@pytest.mark.parametrize("case", GRAD_CASES, ids=lambda c: "x".join(map(str, c)))
def test_single_backward_matches_autograd(case, neg, dtype):
    B, H, U, P, T, K, re_norm, E = case
    A = P ** U
    print(f"decoder backward {case} neg={neg} {dtype}", flush=True)
    g = torch.Generator().manual_seed(int(sum(case) * 17) + int(neg))
    addr = torch.randn(B, H, U, P, T, generator=g).to(dtype)
    pos = torch.randint(0, 5000, (B, T), generator=g)
    D = torch.randn(B, H, K, T, generator=g)
    ops = _ops()
    idx, val = ops.topk_addr_single_forward(addr.to(DEV), E, A, pos.to(DEV), K, re_norm, neg, True)
    grad = ops.topk_addr_single_backward(idx, val, addr.to(DEV), D.to(DEV), E, pos.to(DEV), K, re_norm, neg,
                                         [B, H, U, P, A, T], dtype)
    torch.cuda.synchronize()
    oracle.check_topk_indices(idx.cpu(), addr, E, pos, K)  # the selection (near ties exempt)
    _, rgrad = _reference(addr, E, pos, K, re_norm, True, D, idx=idx.cpu())
    assert grad.dtype == dtype and grad.shape == addr.shape
    err = oracle.rel_err(grad.float().cpu(), rgrad)
    assert err <= _tol(dtype), f"grad rel err {err:.3e}"


def test_pair_backward_and_inactive_addresses():
    """Write and read decoders of one launch (reads stored negated), with
    some addresses inactive (a digit of -inf logits): their gradient is 0."""
    B, H, U, P, T, Kw, Kr, E = 2, 3, 2, 16, 25, 8, 4, 2
    A = P ** U
    g = torch.Generator().manual_seed(123)
    w = torch.randn(B, H, U, P, T, generator=g)
    r = torch.randn(B, H, U, P, T, generator=g)
    w[0, 1, 1, :, 3] = float("-inf")
    r[1, 2, 0, :, 7] = float("-inf")
    pos = torch.randint(0, 5000, (B, T), generator=g)
    D = torch.randn(B, H, Kw + Kr, T, generator=g)
    ops = _ops()
    idx, val = ops.topk_addr_forward(w.to(DEV), r.to(DEV), E, A, pos.to(DEV), Kw, Kr, 0.5, 0.0)
    gw, gr = ops.topk_addr_backward(idx, val, w.to(DEV), r.to(DEV), D.to(DEV), E, pos.to(DEV), Kw, Kr, 0.5, 0.0,
                                    [B, H, U, P, A, T], torch.float32)
    torch.cuda.synchronize()
    ridx_w, rgw = _reference(w, E, pos, Kw, 0.5, True, D[:, :, :Kw])
    ridx_r, rgr = _reference(r, E, pos, Kr, 0.0, True, D[:, :, Kw:])
    live_w = ~torch.isneginf(w).all(dim=-2).any(dim=-2)  # (B, H, T)
    live_r = ~torch.isneginf(r).all(dim=-2).any(dim=-2)
    assert torch.equal(idx.cpu()[:, :, :Kw][live_w.unsqueeze(2).expand(-1, -1, Kw, -1)],
                       ridx_w[live_w.unsqueeze(2).expand(-1, -1, Kw, -1)])
    assert oracle.rel_err(gw.cpu(), rgw) <= 1e-5
    assert oracle.rel_err(gr.cpu(), rgr) <= 1e-5
    assert bool((gw.cpu()[0, 1, :, :, 3] == 0).all()) and bool((gr.cpu()[1, 2, :, :, 7] == 0).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_topk_addr_autograd(dtype):
    """The public ``topk_addr`` is differentiable through the registered backward."""
    from ramnet_ops import topk_addr
    B, H, U, P, T, K, E = 2, 2, 2, 16, 30, 8, 1
    g = torch.Generator().manual_seed(9)
    addr = torch.randn(B, H, U, P, T, generator=g).to(dtype)
    pos = torch.randint(0, 5000, (B, T), generator=g)
    D = torch.randn(B, H, K, T, generator=g)
    a = addr.to(DEV).requires_grad_(True)
    idx, val = topk_addr(a, E, pos.to(DEV), K, 0.25)
    (val * D.to(DEV)).sum().backward()
    torch.cuda.synchronize()
    oracle.check_topk_indices(idx.cpu(), addr, E, pos, K)
    _, rgrad = _reference(addr, E, pos, K, 0.25, True, D, idx=idx.cpu())
    assert oracle.rel_err(a.grad.float().cpu(), rgrad) <= _tol(dtype)


@pytest.mark.parametrize("re_norm", [0.0, 0.5, 1.0])
@pytest.mark.parametrize("neg", [False, True])
def test_inactive_addresses_have_zero_weights_and_gradients(re_norm, neg):
    """The reference's inactive-address test (test_address_numerics.py:58-71)
    through the HIP decoder and its backward: token 0 has every logit -inf,
    token 1 a whole digit of -inf; their weights and gradients are exactly 0
    and everything is finite."""
    from ramnet_ops import topk_addr
    g = torch.Generator().manual_seed(58)
    source = torch.randn(2, 2, 2, 3, 3, generator=g)
    source[..., 0] = float("-inf")
    source[:, :, 0, :, 1] = float("-inf")
    positions = torch.arange(3).expand(2, -1)
    addr = source.to(DEV).requires_grad_(True)
    _, val = topk_addr(addr, 1, positions.to(DEV), 4, re_norm, neg)
    up = torch.randn(val.shape, generator=g).to(DEV)
    grad, = torch.autograd.grad(val, addr, up)
    torch.cuda.synchronize()
    assert bool((val[..., :2] == 0).all()) and bool((grad[..., :2] == 0).all())
    assert bool(torch.isfinite(val).all()) and bool(torch.isfinite(grad).all())


@pytest.mark.parametrize("top_k", [1, 4, 9])
@pytest.mark.parametrize("re_norm", [0.0, 0.5, 1.0])
def test_extreme_logit_gradients(golden, top_k, re_norm):
    """The reference's extreme-logit test (test_address_numerics.py:83-102):
    logits of magnitude ~1000 in float32; weights against the fixture and
    gradients against fp64 autograd of the closed form, on the GPU's selection."""
    from ramnet_ops import topk_addr
    fx = golden("extreme_logits.json")
    src = torch.tensor(fx["addr"], dtype=torch.float64).view(fx["shape"])  # (1, 1, 2, 3, 2)
    positions = torch.arange(2).view(1, 2)
    a = src.float().to(DEV).requires_grad_(True)
    idx, val = topk_addr(a, 0, positions.to(DEV), top_k, re_norm)
    up = torch.randn(val.shape, generator=torch.Generator().manual_seed(top_k)).double()
    grad, = torch.autograd.grad(val, a, up.float().to(DEV))
    torch.cuda.synchronize()
    case = next(c for c in fx["cases"] if c["top_k"] == top_k and c["re_norm"] == re_norm)
    dense = torch.zeros(2, fx["A"], dtype=torch.float64)  # (T, A)
    dense.scatter_(1, idx.cpu()[0, 0].long().t(), val.detach().cpu()[0, 0].double().t())
    assert oracle.rel_err(dense, torch.tensor(case["dense"])) <= 1e-5
    _, rgrad = _reference(src, 0, positions, top_k, re_norm, True, up, idx=idx.cpu())
    assert bool(torch.isfinite(grad).all())
    assert oracle.rel_err(grad.cpu().double(), rgrad) <= 1e-5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_backward_logit_address_high_bit(dtype):
    """The decoder backward bases its buffer resources at each wave's first
    logit and gradient address: logits and gradients whose addresses have bit
    31 of the low word set, and clear, give the same bits as plain
    allocations (the widening of a signed low word would turn such an address
    into a wild one)."""
    from ramnet_ops import _native as nat
    ops = _ops()
    B, H, U, P, T, K, E = 2, 4, 2, 32, 200, 8, 2
    A = P ** U
    g = torch.Generator().manual_seed(37)
    addr = torch.randn(B, H, U, P, T, generator=g).to(dtype).to(DEV)
    pos = torch.randint(0, 1000, (B, T), generator=g).to(DEV)
    idx, val = ops.topk_addr_single_forward(addr, E, A, pos, K, 0.5, False, True)
    dval = torch.randn(B, H, K, T, generator=g).to(DEV)
    ref = ops.topk_addr_single_backward(idx, val, addr, dval, E, pos, K, 0.5, False, [B, H, U, P, A, T], dtype)
    pos32 = pos.to(torch.int32).contiguous()
    nbytes = addr.numel() * addr.element_size()
    pool = torch.empty((1 << 31) + (1 << 23), dtype=torch.uint8, device=DEV)
    base = pool.data_ptr()
    for bit in (True, False):
        offs = [o for o in range(0, pool.numel() - nbytes, 1 << 20) if bool((base + o) & (1 << 31)) == bit]
        xo, go = offs[0], offs[-1]
        print(f"logits at {base + xo:#x}, gradient at {base + go:#x} (bit 31 {'set' if bit else 'clear'})", flush=True)
        x_view = pool[xo:xo + nbytes].view(dtype).view(B, H, U, P, T)
        g_view = pool[go:go + nbytes].view(dtype).view(B, H, U, P, T)
        x_view.copy_(addr)
        nat.call("ramnet_topk_addr_single_backward", idx.data_ptr(), val.data_ptr(), x_view.data_ptr(),
                 dval.data_ptr(), nat.DTYPE_CODES[dtype], B, H, U, P, T, E, A, pos32.data_ptr(), K, 0.5,
                 0, g_view.data_ptr(), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert torch.equal(g_view, ref)
    del pool

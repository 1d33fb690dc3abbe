"""Segment backward on the GPU against fp64 autograd of the dense oracle.

The reference's contract (csrc/ram_attn_segment_parallel.cu:418-606,
ram_attn_ops.cpp:267-310, _cuda_autograd.py:205-287): gradients of the
decoder weights (with respect to the positive weights for reads; zero for
events that do not act), of x and gamma (float32), and of the initial slot
and mass state; the output gradient is taken in x's dtype. The oracle is
torch autograd in float64 through ``oracle.dense_ram_attn`` (the dense
restatement of the reference's torch path), given the same decoded events.
"""
from __future__ import annotations

import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda"
F32, BF16, F16 = torch.float32, torch.bfloat16, torch.float16

CASES = [
    # B, H, U, P, T, C, Kw, Kr, dtype, masked, mass_aware
    (2, 2, 2, 8, 40, 16, 4, 4, F32, False, False),
    (1, 3, 2, 16, 33, 37, 8, 8, F32, True, False),    # odd C: partial channel slices; masked tokens
    (2, 2, 3, 4, 29, 24, 8, 8, F32, True, True),      # mass_aware
    (1, 2, 2, 8, 21, 16, 40, 24, F32, False, True),   # top_k > 32: one 64-event pass
    (1, 1, 2, 16, 13, 8, 100, 70, F32, True, False),  # top_k > 64: two passes
    (1, 2, 2, 16, 1, 16, 8, 8, F32, False, True),     # T = 1
    (2, 2, 2, 16, 40, 64, 8, 8, BF16, True, False),
    (1, 2, 2, 16, 40, 64, 8, 8, F16, False, True),
    (1, 2, 2, 32, 24, 300, 16, 16, F32, False, False),  # C > 16 slices of 4: wider lanes
    (1, 2, 2, 90, 20, 12, 8, 8, F32, True, True),     # A = 8100: 8-channel slices do not fit, 16 event lanes
    (1, 2, 2, 4, 45, 16, 8, 8, F32, False, False),    # A = 16: neighbouring tokens share slots (row reloads)
]


def _ops():
    import ramnet_ops  # noqa: F401  (registers torch.ops.ramnet_ops.*)
    return torch.ops.ramnet_ops


def _tol(dtype):
    return 1e-5 if dtype == F32 else 2e-2


def _inputs(B, H, U, P, T, C, Kw, Kr, dtype, masked, seed):
    g = torch.Generator().manual_seed(seed)
    A = P ** U
    w = (1.5 * torch.randn(B, H, U, P, T, generator=g)).to(dtype)
    r = (1.5 * torch.randn(B, H, U, P, T, generator=g)).to(dtype)
    pos = torch.randint(0, 4 * A, (B, T), generator=g)
    x = torch.randn(B, H, T, C, generator=g).to(dtype)
    gamma = (2.0 * torch.randn(B, H, T, generator=g)).to(dtype)
    slot = 0.5 * torch.randn(B, H, A, C, generator=g)
    mass = torch.rand(B, H, A, generator=g) + 0.05
    mask = (torch.rand(B, T, generator=g) > 0.3) if masked else None
    Dy = torch.randn(B, H, T, C, generator=g).to(dtype)
    Ds = torch.randn(B, H, A, C, generator=g)
    Dm = torch.randn(B, H, A, generator=g)
    return dict(w=w, r=r, pos=pos, x=x, gamma=gamma, slot=slot, mass=mass, mask=mask, Dy=Dy, Ds=Ds, Dm=Dm, A=A)


def _oracle(idx, val, x, gamma, slot, mass, mask, Dy, Ds, Dm, Kw, Kr, mass_aware, eps, U, P):
    """fp64 autograd of sum(y Dy) + sum(slot' Ds) + sum(mass' Dm) given the decoded events."""
    B, H, T, C = x.shape
    wv = val[:, :, :Kw].double().clone().requires_grad_(True)
    rv = (-val[:, :, Kw:]).double().clone().requires_grad_(True)  # positive read weights
    x64 = x.double().requires_grad_(True)
    g64 = gamma.double().requires_grad_(True)
    s64 = slot.double().requires_grad_(True)
    m64 = mass.double().requires_grad_(True)
    dummy = torch.zeros(B, H, U, P, T, dtype=torch.float64)
    y, s, m = oracle.dense_ram_attn(dummy, dummy, x64, g64, s64, m64, mask, 0, None, (Kw, Kr), (0.0, 0.0),
                                    mass_aware, eps, decoded=(idx[:, :, :Kw], wv, idx[:, :, Kw:], -rv))
    keep = torch.ones(B, T, dtype=torch.float64) if mask is None else mask.double()
    loss = (y * Dy.double() * keep[:, None, :, None]).sum() + (s * Ds.double()).sum() + (m * Dm.double()).sum()
    loss.backward()
    dval = torch.cat([wv.grad, rv.grad], dim=2)
    dval = dval.masked_fill(val == 0, 0)  # events that do not act carry no gradient (the reference skips them)
    return dval, x64.grad, g64.grad, s64.grad, m64.grad


def _check(name, got, ref, tol):
    err = oracle.rel_err(got.cpu().double(), ref)
    print(f"  {name}: rel {err:.2e}", flush=True)
    assert err <= tol, f"{name}: rel err {err:.3e} > {tol}"


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_segment_backward_matches_oracle(case):
    B, H, U, P, T, C, Kw, Kr, dtype, masked, mass_aware = case
    ops = _ops()
    print(f"segment backward case {case}", flush=True)
    d = _inputs(B, H, U, P, T, C, Kw, Kr, dtype, masked, seed=B * 1000 + T * 10 + C + Kw)
    A = d["A"]
    idx, val = ops.topk_addr_forward(d["w"].to(DEV), d["r"].to(DEV), 1, A, d["pos"].to(DEV).int(), Kw, Kr, 0.0, 0.0)
    mask = None if d["mask"] is None else d["mask"].to(DEV)
    got = ops.topk_segment_backward(idx, val, d["x"].to(DEV), d["gamma"].to(DEV), d["slot"].to(DEV),
                                    d["mass"].to(DEV), mask, d["Dy"].to(DEV), d["Ds"].to(DEV), d["Dm"].to(DEV),
                                    Kw, Kr, mass_aware, 1e-12)
    torch.cuda.synchronize()
    ref = _oracle(idx.cpu(), val.cpu(), d["x"], d["gamma"], d["slot"], d["mass"], d["mask"], d["Dy"], d["Ds"],
                  d["Dm"], Kw, Kr, mass_aware, 1e-12, U, P)
    tol = _tol(dtype)
    for name, g, r in zip(("D_addr_val", "D_x", "D_gamma", "D_slot", "D_mass"), got, ref):
        _check(name, g, r, tol)
    # the output gradient of masked tokens is ignored: zeroing it changes nothing
    if mask is not None:
        Dy0 = d["Dy"].masked_fill(~d["mask"][:, None, :, None], 0).to(DEV)
        again = ops.topk_segment_backward(idx, val, d["x"].to(DEV), d["gamma"].to(DEV), d["slot"].to(DEV),
                                          d["mass"].to(DEV), mask, Dy0, d["Ds"].to(DEV), d["Dm"].to(DEV), Kw, Kr,
                                          mass_aware, 1e-12)
        for a, b in zip(got, again):
            assert torch.equal(a, b)


WIDE_CASES = [
    # B, H, U, P, T, C, Kw, Kr, dtype, masked, mass_aware: slot spaces beyond
    # 13652, where the forward replay's tag tables run in slot ranges
    (1, 2, 7, 4, 50, 8, 8, 8, F32, False, True),      # A = 16384, mass_aware
    (1, 2, 3, 32, 60, 8, 8, 8, F32, True, False),     # A = 32768, masked tokens
    (1, 1, 3, 32, 50, 12, 16, 8, F32, False, True),   # A = 32768, Kw != Kr, mass_aware
    (1, 1, 5, 8, 40, 8, 100, 70, F32, True, True),    # A = 32768, two 64-event passes
    (1, 2, 3, 32, 40, 8, 8, 8, BF16, False, False),
]


@pytest.mark.parametrize("case", WIDE_CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_segment_backward_wide_slot_space(case):
    """The segment backward beyond A = 13652 (the reference's is bounded only
    by int32): the forward mass replay in record-keeping mode split into slot
    ranges (mass-aware weights scaled per token afterwards), the slice scan
    with one channel per wave, against the fp64 state-reconstruction oracle
    on the GPU's events."""
    B, H, U, P, T, C, Kw, Kr, dtype, masked, mass_aware = case
    ops = _ops()
    print(f"wide segment backward case {case}", flush=True)
    d = _inputs(B, H, U, P, T, C, Kw, Kr, dtype, masked, seed=B * 1000 + T * 10 + C + Kw + 7)
    A = d["A"]
    idx, val = ops.topk_addr_forward(d["w"].to(DEV), d["r"].to(DEV), 1, A, d["pos"].to(DEV).int(), Kw, Kr, 0.0, 0.0)
    mask = None if d["mask"] is None else d["mask"].to(DEV)
    got = ops.topk_segment_backward(idx, val, d["x"].to(DEV), d["gamma"].to(DEV), d["slot"].to(DEV),
                                    d["mass"].to(DEV), mask, d["Dy"].to(DEV), d["Ds"].to(DEV), d["Dm"].to(DEV),
                                    Kw, Kr, mass_aware, 1e-12)
    torch.cuda.synchronize()
    got = [t.cpu() for t in got]
    wi, wv, ri, rv = oracle.split_events(idx.cpu(), val.cpu(), Kw)
    ref = oracle.sparse_gsu_backward_f64(wi, wv, ri, rv, d["x"].double(), d["gamma"].double(), d["slot"], d["mass"],
                                         d["Dy"].double(), d["Ds"], d["Dm"], d["mask"], mass_aware, 1e-12)
    tol = _tol(dtype)
    names = ("D_w", "D_r", "D_x", "D_gamma", "D_init_slot", "D_init_mass")
    mine = (got[0][:, :, :Kw], got[0][:, :, Kw:], got[1], got[2], got[3], got[4])
    for name, a, b in zip(names, mine, ref):
        _check(name, a, torch.as_tensor(b), tol)


def test_segment_backward_deterministic_and_optional_grads():
    """Two calls give identical bits; absent final-state gradients act as zeros."""
    ops = _ops()
    B, H, U, P, T, C, K = 2, 4, 2, 16, 200, 64, 8
    d = _inputs(B, H, U, P, T, C, K, K, BF16, True, seed=7)
    A = d["A"]
    idx, val = ops.topk_addr_forward(d["w"].to(DEV), d["r"].to(DEV), 2, A, d["pos"].to(DEV).int(), K, K, 0.0, 0.0)
    args = (idx, val, d["x"].to(DEV), d["gamma"].to(DEV), d["slot"].to(DEV), d["mass"].to(DEV), d["mask"].to(DEV),
            d["Dy"].to(DEV))
    a = ops.topk_segment_backward(*args, None, None, K, K, True, 1e-12)
    b = ops.topk_segment_backward(*args, None, None, K, K, True, 1e-12)
    z = ops.topk_segment_backward(*args, torch.zeros_like(d["Ds"]).to(DEV), torch.zeros_like(d["Dm"]).to(DEV),
                                  K, K, True, 1e-12)
    for u, v, w in zip(a, b, z):
        assert torch.equal(u, v)
        assert torch.equal(u, w)


def _vals_from_logits(a64, idx, E, pos, K, re_norm):
    """The decoder's weights in fp64 as a differentiable function of the
    logits, for a given (GPU) selection."""
    B, H, U, P, T = a64.shape
    A = P ** U
    scores = oracle.content_scores(oracle.log_softmax_digits(a64, torch.float64))  # (B, H, T, A)
    heads = torch.arange(H).view(1, H, 1, 1)
    shift = (heads < E).long() * pos.long().view(B, 1, 1, T)
    content = torch.remainder(idx.long() % A + shift, A)  # (B, H, K, T)
    s = scores.gather(-1, content.permute(0, 1, 3, 2))  # (B, H, T, K)
    if re_norm != 0:
        s = s - re_norm * s.logsumexp(dim=-1, keepdim=True)
    return s.exp().permute(0, 1, 3, 2)


@pytest.mark.parametrize("T,mass_aware,masked,dtype", [(48, False, True, F32), (37, True, False, F32),
                                                      (1, False, False, F32), (40, True, True, BF16)])
def test_api_gradients_match_oracle(T, mass_aware, masked, dtype):
    """random_access_memory_attention with inputs that require grad: the
    composed decoder + segment backward against fp64 autograd of the dense
    reference, down to the address logits."""
    from ramnet_ops import random_access_memory_attention
    print(f"api gradients T={T} mass_aware={mass_aware} masked={masked} {dtype}", flush=True)
    B, H, U, P, C, K, E = 2, 3, 2, 8, 24, 6, 2
    re = (0.5, 0.25)
    d = _inputs(B, H, U, P, T, C, K, K, dtype, masked, seed=T + 100 * int(mass_aware))
    A = d["A"]
    leaves = {k: d[k].to(DEV).requires_grad_(True) for k in ("w", "r", "x", "gamma", "slot", "mass")}
    mask = None if d["mask"] is None else d["mask"].to(DEV)
    y, (slot, mass) = random_access_memory_attention(
        leaves["w"].permute(0, 4, 1, 2, 3), leaves["r"].permute(0, 4, 1, 2, 3), leaves["x"].permute(0, 2, 1, 3),
        leaves["gamma"].permute(0, 2, 1), init_ram=(leaves["slot"], leaves["mass"]), mask=mask, embed_num=E,
        position_ids=d["pos"].to(DEV), top_k=K, top_k_re_norm=re, mass_aware=mass_aware)
    loss = (y.float() * d["Dy"].permute(0, 2, 1, 3).float().to(DEV)).sum() + (slot * d["Ds"].to(DEV)).sum() \
        + (mass * d["Dm"].to(DEV)).sum()
    loss.backward()
    torch.cuda.synchronize()

    # the GPU's selection, then the fp64 reference as a function of the logits
    ops = _ops()
    idx, _ = ops.topk_addr_forward(d["w"].to(DEV), d["r"].to(DEV), E, A, d["pos"].to(DEV).int(), K, K, *re)
    idx = idx.cpu()
    w64 = d["w"].double().requires_grad_(True)
    r64 = d["r"].double().requires_grad_(True)
    x64 = d["x"].double().requires_grad_(True)
    g64 = d["gamma"].double().requires_grad_(True)
    s64 = d["slot"].double().requires_grad_(True)
    m64 = d["mass"].double().requires_grad_(True)
    wv = _vals_from_logits(w64, idx[:, :, :K], E, d["pos"], K, re[0])
    rv = _vals_from_logits(r64, idx[:, :, K:], E, d["pos"], K, re[1])
    dummy = torch.zeros(B, H, U, P, T, dtype=torch.float64)
    ry, rs, rm = oracle.dense_ram_attn(dummy, dummy, x64, g64, s64, m64, d["mask"], 0, None, (K, K), (0.0, 0.0),
                                       mass_aware, 1e-12, decoded=(idx[:, :, :K], wv, idx[:, :, K:], -rv))
    keep = torch.ones(B, T, dtype=torch.float64) if d["mask"] is None else d["mask"].double()
    # the op casts y to the activation dtype: its gradient arrives in that dtype too
    Dy = d["Dy"].float().to(dtype).double()
    ref_loss = (ry * Dy * keep[:, None, :, None]).sum() + (rs * d["Ds"].double()).sum() + (rm * d["Dm"].double()).sum()
    ref_loss.backward()
    tol = _tol(dtype)
    for name, leaf, ref in (("w_addr", leaves["w"], w64), ("r_addr", leaves["r"], r64), ("values", leaves["x"], x64),
                            ("gamma", leaves["gamma"], g64), ("slot", leaves["slot"], s64),
                            ("mass", leaves["mass"], m64)):
        _check(name, leaf.grad, ref.grad, tol)


def test_inplace_with_grad_raises():
    from ramnet_ops import random_access_memory_attention
    B, H, U, P, T, C = 1, 2, 2, 8, 8, 16
    A = P ** U
    w = torch.randn(B, T, H, U, P, device=DEV, requires_grad=True)
    slot = torch.zeros(B, H, A, C, device=DEV)
    mass = torch.full((B, H, A), 1.0 / A, device=DEV)
    with pytest.raises(AssertionError, match="inplace"):
        random_access_memory_attention(w, w, torch.randn(B, T, H, C, device=DEV), init_ram=(slot, mass),
                                       top_k=4, inplace=True)


@pytest.mark.parametrize("mass_aware", [False, True])
def test_config2_full_size_backward_heads(mass_aware):
    """Config 2 at full size (B=8, H=16, T=4096, d_v=128, A=1024, K=8, bf16):
    the whole backward on the GPU, then two heads (first and last) against the
    fp64 state-reconstruction oracle on the GPU's events. Heads are
    independent, so each head's gradients are complete on its own."""
    from ram_cases import projected_logits
    ops = _ops()
    B, H, U, P, T, C, K = 8, 16, 2, 32, 4096, 128, 8
    A = P ** U
    print(f"config 2 full-size backward, mass_aware={mass_aware}", flush=True)
    w, r = projected_logits(B, H, U, P, T, 128, seed=2)
    g = torch.Generator().manual_seed(21)
    x = torch.randn(B, H, T, C, generator=g).to(torch.bfloat16)
    gamma = torch.sigmoid(torch.randn(B, H, T, generator=g) - 1).to(torch.bfloat16)
    pos = torch.arange(T).view(1, T).expand(B, T)
    Dy = torch.randn(B, H, T, C, generator=g).to(torch.bfloat16)
    Ds = torch.randn(B, H, A, C, generator=g)
    Dm = torch.randn(B, H, A, generator=g)
    slot0 = torch.zeros(B, H, A, C)
    mass0 = torch.full((B, H, A), 1.0 / A)
    idx, val = ops.topk_addr_forward(w.to(DEV), r.to(DEV), H // 2, A, pos.to(DEV), K, K, 0.0, 0.0)
    got = ops.topk_segment_backward(idx, val, x.to(DEV), gamma.to(DEV), slot0.to(DEV), mass0.to(DEV), None,
                                    Dy.to(DEV), Ds.to(DEV), Dm.to(DEV), K, K, mass_aware, 1e-12)
    torch.cuda.synchronize()
    got = [t.cpu() for t in got]
    idx_c, val_c = idx.cpu(), val.cpu()
    heads = ((0, 0), (7, 15))
    sel = lambda t: torch.stack([t[b, h] for b, h in heads]).unsqueeze(1)  # (2, 1, ...)
    local = torch.stack([idx_c[b, h] - (b * H + h) * A for b, h in heads]).unsqueeze(1)
    vsel = sel(val_c)
    wi, wv, ri, rv = local[:, :, :K], vsel[:, :, :K], local[:, :, K:], -vsel[:, :, K:]
    ref = oracle.sparse_gsu_backward_f64(wi, wv, ri, rv, sel(x).double(), sel(gamma).double(), sel(slot0),
                                         sel(mass0), sel(Dy).double(), sel(Ds), sel(Dm), None, mass_aware, 1e-12,
                                         encoded=False)
    gval = sel(got[0])
    names = ("D_w", "D_r", "D_x", "D_gamma", "D_init_slot", "D_init_mass")
    mine = (gval[:, :, :K], gval[:, :, K:], sel(got[1]), sel(got[2]), sel(got[3]), sel(got[4]))
    for name, a, b in zip(names, mine, ref):
        _check(name, a, torch.as_tensor(b), 1e-5)


def test_config4_full_size_backward_heads():
    """Config 4 at full size (B=4, H=8, T=8192, U=3, P=16 -> A=4096, K=16,
    bf16): the backward on the GPU (16-event lanes, 4-channel slices), two
    heads against the fp64 state-reconstruction oracle on the GPU's events."""
    from ram_cases import projected_logits
    ops = _ops()
    B, H, U, P, T, C, K, E = 4, 8, 3, 16, 8192, 128, 16, 4
    A = P ** U
    print("config 4 full-size backward", flush=True)
    w, r = projected_logits(B, H, U, P, T, 128, seed=4, dtype=torch.float32)
    w, r = w.to(torch.bfloat16), r.to(torch.bfloat16)
    g = torch.Generator().manual_seed(41)
    x = torch.randn(B, H, T, C, generator=g).to(torch.bfloat16)
    gamma = torch.sigmoid(torch.randn(B, H, T, generator=g)).to(torch.bfloat16)
    pos = torch.arange(T).view(1, T).expand(B, T)
    Dy = torch.randn(B, H, T, C, generator=g).to(torch.bfloat16)
    slot0 = torch.zeros(B, H, A, C)
    mass0 = torch.full((B, H, A), 1.0 / A)
    idx, val = ops.topk_addr_forward(w.to(DEV), r.to(DEV), E, A, pos.to(DEV), K, K, 0.0, 0.0)
    got = ops.topk_segment_backward(idx, val, x.to(DEV), gamma.to(DEV), slot0.to(DEV), mass0.to(DEV), None,
                                    Dy.to(DEV), None, None, K, K, False, 1e-12)
    torch.cuda.synchronize()
    got = [t.cpu() for t in got]
    idx_c, val_c = idx.cpu(), val.cpu()
    heads = ((0, 0), (3, 7))
    sel = lambda t: torch.stack([t[b, h] for b, h in heads]).unsqueeze(1)  # (2, 1, ...)
    local = torch.stack([idx_c[b, h] - (b * H + h) * A for b, h in heads]).unsqueeze(1)
    vsel = sel(val_c)
    ref = oracle.sparse_gsu_backward_f64(local[:, :, :K], vsel[:, :, :K], local[:, :, K:], -vsel[:, :, K:],
                                         sel(x).double(), sel(gamma).double(), sel(slot0), sel(mass0),
                                         sel(Dy).double(), None, None, None, False, 1e-12, encoded=False)
    gval = sel(got[0])
    names = ("D_w", "D_r", "D_x", "D_gamma", "D_init_slot", "D_init_mass")
    mine = (gval[:, :, :K], gval[:, :, K:], sel(got[1]), sel(got[2]), sel(got[3]), sel(got[4]))
    for name, a, b in zip(names, mine, ref):
        _check(name, a, torch.as_tensor(b), 1e-5)


RE_NORMS = [(0.0, 0.0), (1.0, 1.0), (0.25, 0.75), (0.75, 0.25)]


def _chunk_case(B, H, U, P, C, T, seed, masked):
    g = torch.Generator().manual_seed(seed)
    A = P ** U

    def rn(*s):
        return torch.randn(*s, generator=g).to(DEV)

    d = dict(w=rn(B, H, U, P, T), r=rn(B, H, U, P, T), x=rn(B, H, T, C), gamma=0.2 * rn(B, H, T),
             slot=rn(B, H, A, C), mass=(torch.rand(B, H, A, generator=g) + 0.1).to(DEV),
             d_y=rn(B, H, T, C), d_slot=rn(B, H, A, C), d_mass=rn(B, H, A), mask=None,
             pos=torch.arange(T, device=DEV).view(1, T).expand(B, T))
    if masked:
        mask = torch.ones(B, T, dtype=torch.bool, device=DEV)
        mask[:, 22:44] = False  # a whole chunk carries the state without updates
        mask[0, ::5] = False
        mask[1, 1::7] = False
        d.update(mask=mask, pos=(mask.long().cumsum(-1) - 1).masked_fill(~mask, 0),
                 d_y=d["d_y"] * mask[:, None, :, None])
    return d


def _chunked_run(d, chunk, top_k, re_norm, mass_aware):
    """Outputs and the gradients of all six inputs with the sequence run in
    chunks, each from the previous chunk's post state
    (ram_attention_helpers.py:114-190)."""
    from ramnet_ops.impl.cuda_impl import _cuda_ram_attn
    T = d["x"].shape[2]
    inputs = [d[k].detach().clone().requires_grad_() for k in ("w", "r", "x", "gamma", "slot", "mass")]
    wa, ra, xa, ga, slot, mass = inputs
    ys = []
    for s in range(0, T, chunk):
        st = slice(s, s + chunk)
        y, slot, mass = _cuda_ram_attn(wa[..., st], ra[..., st], xa[..., st, :], ga[..., st], slot, mass,
                                       None if d["mask"] is None else d["mask"][:, st], 1, d["pos"][:, st], top_k,
                                       re_norm, mass_aware, 1e-12, False)
        ys.append(y)
    outs = (torch.cat(ys, dim=-2), slot, mass)
    grads = torch.autograd.grad(outs, inputs, (d["d_y"], d["d_slot"], d["d_mass"]))
    if d["mask"] is not None:
        outs = (outs[0] * d["mask"][:, None, :, None], *outs[1:])
    return outs, grads


def _assert_chunked_matches_full(d, chunks, top_k, re_norm, mass_aware, tol=1e-4):
    full, g_full = _chunked_run(d, d["x"].shape[2], top_k, re_norm, mass_aware)
    for chunk in chunks:
        outs, grads = _chunked_run(d, chunk, top_k, re_norm, mass_aware)
        for a, b in zip((*outs, *grads), (*full, *g_full)):
            torch.testing.assert_close(a, b, atol=tol, rtol=tol)


@pytest.mark.parametrize("masked", [False, True], ids=["unmasked", "masked"])
@pytest.mark.parametrize("re_norm", RE_NORMS)
@pytest.mark.parametrize("mass_aware", [False, True], ids=["plain", "mass_aware"])
def test_chunked_state_and_gradients_match_full(masked, re_norm, mass_aware):
    """The reference's chunk contract with gradients
    (test_ram_attention_behavior.py:55-75): the sequence run in chunks of 22,
    32 and 33 tokens gives the full run's outputs (y on valid tokens) and the
    same gradients of all six inputs; with a mask, a whole chunk of tokens
    carries the state without updates."""
    d = _chunk_case(2, 4, 3, 4, 8, 65, seed=55, masked=masked)
    _assert_chunked_matches_full(d, (22, 32, 33), (4, 8), re_norm, mass_aware)


@pytest.mark.parametrize("top_k", [(4, 4), (8, 8), (4, 12), (16, 16), (32, 32), (64, 64), (128, 128)],
                         ids=lambda k: "k{}x{}".format(*k))
@pytest.mark.parametrize("re_norm", RE_NORMS)
def test_top_k_range_and_long_sequence(top_k, re_norm):
    """The reference's top-K range on a long sequence
    (test_ram_attention_behavior.py:77-88, ram_attention_helpers.py:14-15):
    A = 4^5 = 1024 slots, 16 channels, T = 1024 in chunks of 128 against the
    full run, outputs and gradients, for every top-K and re-norm setting."""
    print(f"long sequence top_k={top_k} re_norm={re_norm}", flush=True)
    d = _chunk_case(2, 4, 5, 4, 16, 1024, seed=77, masked=False)
    _assert_chunked_matches_full(d, (128,), top_k, re_norm, False)

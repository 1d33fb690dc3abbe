"""The reference's own CUDA-against-torch numerics grid, run through this
build's GPU path against the CPU oracle.

Mirrors tests/ops/test_ram_attention_numerics.py of the reference (its
SHAPE_CASES, TOP_K_RE_NORM_SETTINGS, mass_aware, the mask and shifted-position
modes, the sequence boundaries and the low-precision runs) with inputs built
as its make_ram_case builds them (tests/ops/ram_attention_helpers.py:46-94:
batch 2, 4 heads, CAPE on 4 heads, top-K (8, 8), random initial state,
random gradients of y and of the final state). Where the reference compares
its CUDA op with its torch path, this compares the HIP op with:

* outputs: the dense fp64 restatement of the torch path (``dense_ram_attn``,
  its own decode) when the fp64 ranking has no near-tie in the GPU's
  selection, else the fp64 event loop on the GPU's selection;
* gradients of all six inputs: the fp64 state-reconstruction backward on the
  GPU's selection, chained through fp64 autograd of the decoder weights down
  to the address logits.

The in-place forms (``ram_attn_forward_``, ``topk_segment_forward_``) are
checked the same way from a random non-zero state with masks.

Bars: indices bit-exact except fp64 ties within 1e-6; fp32 rel <= 1e-5;
bfloat16 / float16 rel <= 2e-2 (max|a-b| / max|b| per tensor; y and the
time-indexed gradients on valid tokens only).
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import pytest
import torch

import oracle
from test_gpu_segment_backward import _vals_from_logits

pytestmark = pytest.mark.gpu

DEV = "cuda"
FP32_TOL = 1e-5
LOW_TOL = 2e-2
EMBED_NUM = 4
TOP_K = (8, 8)
EPS = 1e-12
# U, P, C, T (reference SHAPE_CASES: partial template widths and a long sequence)
SHAPE_CASES = ((4, 3, 29, 1024), (4, 5, 47, 33), (4, 7, 65, 128), (5, 4, 32, 1024))
TOP_K_RE_NORM_SETTINGS = ((0.0, 0.0), (1.0, 1.0), (0.25, 0.75), (0.75, 0.25))
# reference ram_attention_helpers.py:14
TOP_K_SETTINGS = ((4, 4), (8, 8), (4, 12), (16, 16), (32, 32), (64, 64), (128, 128))


@dataclass(frozen=True)
class Case:
    w_addr: torch.Tensor      # (B, H, U, P, T)
    r_addr: torch.Tensor
    values: torch.Tensor      # (B, H, T, C)
    gamma: torch.Tensor       # (B, H, T)
    init_slot: torch.Tensor   # (B, H, A, C) float32
    init_mass: torch.Tensor   # (B, H, A) float32
    d_y: torch.Tensor
    d_slot: torch.Tensor
    d_mass: torch.Tensor
    position_ids: torch.Tensor  # (B, T) int64
    mask: torch.Tensor | None   # (B, T) bool


def make_ram_case(*, batch=2, heads=4, order=5, radix=4, channels=32, seq_len=1024, masked=True, seed=0) -> Case:
    """The reference's case layout (ram_attention_helpers.py:46-94), seeded, on the CPU."""
    g = torch.Generator().manual_seed(seed)
    slots = radix ** order

    def rn(*s):
        return torch.randn(*s, generator=g)
    w = rn(batch, heads, order, radix, seq_len)
    r = rn(batch, heads, order, radix, seq_len)
    values = rn(batch, heads, seq_len, channels)
    gamma = 0.2 * rn(batch, heads, seq_len)
    slot = rn(batch, heads, slots, channels)
    mass = torch.rand(batch, heads, slots, generator=g) + 0.1
    d_y = rn(batch, heads, seq_len, channels)
    d_slot = rn(batch, heads, slots, channels)
    d_mass = rn(batch, heads, slots)
    if masked:
        mask = torch.ones(batch, seq_len, dtype=torch.bool)
        pad = max(1, seq_len // 8)
        mid = seq_len // 2 - pad // 2
        mask[:, :pad] = False
        mask[:, mid:mid + pad] = False
        mask[:, -pad:] = False
        pos = (mask.long().cumsum(-1) - 1).masked_fill(~mask, 0)
    else:
        mask = None
        pos = torch.arange(seq_len).view(1, seq_len).expand(batch, -1).contiguous()
    return Case(w, r, values, gamma, slot, mass, d_y, d_slot, d_mass, pos, mask)


def cast_case(case: Case, dtype) -> Case:
    """Activations, logits and the output gradient in ``dtype``; the state stays fp32."""
    return replace(case, w_addr=case.w_addr.to(dtype), r_addr=case.r_addr.to(dtype), values=case.values.to(dtype),
                   gamma=case.gamma.to(dtype), d_y=case.d_y.to(dtype))


def run_gpu(case: Case, *, top_k=TOP_K, re_norm=(0.0, 0.0), mass_aware=False, chunk=None, grad=True):
    """The HIP path as the reference's gather_ram_result drives its backends
    (ram_attention_helpers.py:114-190): the sequence in chunks from the
    previous chunk's post state, then autograd of (y, slot, mass) against
    (d_y masked, d_slot, d_mass). Returns fwd (y, slot, mass) and the six
    input gradients (or None), on the CPU."""
    from ramnet_ops.impl.cuda_impl import _cuda_ram_attn
    d = {k: getattr(case, k).to(DEV) for k in ("w_addr", "r_addr", "values", "gamma", "init_slot", "init_mass")}
    inputs = [d[k].detach().clone().requires_grad_(grad) for k in d]
    w, r, x, gm, slot, mass = inputs
    mask = None if case.mask is None else case.mask.to(DEV)
    pos = case.position_ids.to(DEV)
    T = x.shape[-2]
    chunk = T if chunk is None else chunk
    ys = []
    with torch.set_grad_enabled(grad):
        for s in range(0, T, chunk):
            st = slice(s, s + chunk)
            y, slot, mass = _cuda_ram_attn(w[..., st], r[..., st], x[..., st, :], gm[..., st], slot, mass,
                                           None if mask is None else mask[:, st], EMBED_NUM, pos[:, st], top_k,
                                           re_norm, mass_aware, EPS, False)
            ys.append(y)
        fwd = (torch.cat(ys, dim=-2), slot, mass)
        grads = None
        if grad:
            dy = case.d_y.to(DEV)
            if mask is not None:
                dy = dy * mask[:, None, :, None].to(dy.dtype)
            grads = torch.autograd.grad(fwd, inputs, (dy, case.d_slot.to(DEV), case.d_mass.to(DEV)))
    torch.cuda.synchronize()
    fwd = tuple(t.detach().cpu() for t in fwd)
    return fwd, None if grads is None else tuple(t.cpu() for t in grads)


def gpu_selection(case: Case, top_k, re_norm):
    """The HIP decoder's indices (B, H, K, T) for both addresses, checked
    against the fp64 ranking; returns them and the number of exempt ties."""
    from ramnet_ops import topk_addr
    out, exempt = [], 0
    for lg, k, rn in ((case.w_addr, top_k[0], re_norm[0]), (case.r_addr, top_k[1], re_norm[1])):
        idx, _ = topk_addr(lg.to(DEV), EMBED_NUM, case.position_ids.to(DEV), k, rn)
        idx = idx.cpu()
        st = oracle.check_topk_indices(idx, lg.float(), EMBED_NUM, case.position_ids, k)
        exempt += st["exempt_slots"]
        out.append(idx)
    return out[0], out[1], exempt


def run_oracle(case: Case, *, top_k=TOP_K, re_norm=(0.0, 0.0), mass_aware=False, grad=True, dense=False):
    """fp64 outputs (and gradients) for the GPU's selection; with ``dense``
    and no near-tie in that selection, the outputs come from the dense
    restatement's own decode instead."""
    wi, ri, exempt = gpu_selection(case, top_k, re_norm)
    B, H, U, P, T = case.w_addr.shape
    w64 = case.w_addr.double().requires_grad_(grad)
    r64 = case.r_addr.double().requires_grad_(grad)
    wv = _vals_from_logits(w64, wi, EMBED_NUM, case.position_ids, top_k[0], re_norm[0])
    rv = _vals_from_logits(r64, ri, EMBED_NUM, case.position_ids, top_k[1], re_norm[1])
    x64, g64 = case.values.double(), case.gamma.double()
    if dense and exempt == 0:
        y, slot, mass = oracle.dense_ram_attn(w64.detach(), r64.detach(), x64, g64, case.init_slot.double(),
                                              case.init_mass.double(), case.mask, EMBED_NUM, case.position_ids,
                                              top_k, re_norm, mass_aware, EPS)
    else:
        y, slot, mass = oracle.sparse_gsu_f64(wi, wv.detach(), ri, rv.detach(), x64, g64, case.init_slot,
                                              case.init_mass, case.mask, mass_aware, EPS)
    fwd = tuple(torch.as_tensor(t).double() for t in (y, slot, mass))
    if not grad:
        return fwd, None
    dy = case.d_y.double()
    d_wv, d_rv, d_x, d_g, d_s, d_m = oracle.sparse_gsu_backward_f64(
        wi, wv.detach(), ri, rv.detach(), x64, g64, case.init_slot, case.init_mass, dy, case.d_slot, case.d_mass,
        case.mask, mass_aware, EPS)
    d_w, d_r = torch.autograd.grad((wv, rv), (w64, r64), (torch.as_tensor(d_wv), torch.as_tensor(d_rv)))
    grads = (d_w, d_r) + tuple(torch.as_tensor(t) for t in (d_x, d_g, d_s, d_m))
    return fwd, grads


def assert_pairs(label, got, ref, mask, tol):
    """Per-tensor relative error; y and the time-indexed gradients on valid tokens."""
    (gy, gs, gm), ggr = got
    (ry, rs, rm), rgr = ref
    time_dim = {"y": -2, "D_w": -1, "D_r": -1, "D_x": -2, "D_gamma": -1}
    pairs = [("y", gy, ry), ("slot", gs, rs), ("mass", gm, rm)]
    if ggr is not None:
        pairs += list(zip(("D_w", "D_r", "D_x", "D_gamma", "D_slot", "D_mass"), ggr, rgr))
    for name, a, b in pairs:
        a, b = a.double(), b.double()
        if mask is not None and name in time_dim:
            keep = mask[0]
            a, b = a.index_select(time_dim[name] % a.dim(), keep.nonzero()[:, 0]), \
                b.index_select(time_dim[name] % b.dim(), keep.nonzero()[:, 0])
        err = oracle.rel_err(a, b)
        assert err <= tol, f"{label}: {name} rel err {err:.3e} > {tol}"
    if mask is not None:
        assert bool((gy[:, :, ~mask[0]] == 0).all()), f"{label}: masked tokens must read 0"


@pytest.mark.parametrize("mass_aware", [False, True], ids=["plain", "mass_aware"])
@pytest.mark.parametrize("re_norm", TOP_K_RE_NORM_SETTINGS, ids=lambda r: "r{}-{}".format(*r))
@pytest.mark.parametrize("shape", SHAPE_CASES, ids=lambda s: "U{}P{}C{}T{}".format(*s))
def test_fp32_matches_oracle(shape, re_norm, mass_aware):
    """test_ram_attention_numerics.py:31-41: outputs and all six gradients."""
    U, P, C, T = shape
    print(f"grid fp32 U={U} P={P} C={C} T={T} re_norm={re_norm} mass_aware={mass_aware}", flush=True)
    case = make_ram_case(order=U, radix=P, channels=C, seq_len=T, masked=False, seed=sum(shape))
    opts = dict(re_norm=re_norm, mass_aware=mass_aware)
    assert_pairs("fp32", run_gpu(case, **opts), run_oracle(case, dense=True, **opts), None, FP32_TOL)


def _mode_cases():
    source = make_ram_case(order=3, channels=16, seq_len=65, seed=65)
    shifted = replace(source, position_ids=(source.position_ids * 3 + 11).masked_fill(~source.mask, 0))
    return {"unmasked": replace(source, mask=None), "masked": source, "shifted": shifted}


@pytest.mark.parametrize("mass_aware", [False, True], ids=["plain", "mass_aware"])
@pytest.mark.parametrize("re_norm", TOP_K_RE_NORM_SETTINGS, ids=lambda r: "r{}-{}".format(*r))
@pytest.mark.parametrize("mode", ["unmasked", "masked", "shifted"])
def test_fp32_mask_and_position_modes(mode, re_norm, mass_aware):
    """test_ram_attention_numerics.py:43-58: masks and shifted CAPE positions."""
    case = _mode_cases()[mode]
    print(f"grid mode {mode} re_norm={re_norm} mass_aware={mass_aware}", flush=True)
    opts = dict(re_norm=re_norm, mass_aware=mass_aware)
    assert_pairs(mode, run_gpu(case, **opts), run_oracle(case, dense=True, **opts), case.mask, FP32_TOL)


@pytest.mark.parametrize("mass_aware", [False, True], ids=["plain", "mass_aware"])
@pytest.mark.parametrize("T", [1, 31, 32, 33])
def test_fp32_sequence_boundaries(T, mass_aware):
    """test_ram_attention_numerics.py:60-66: T around the 32-token record padding, top-K (4, 8)."""
    case = make_ram_case(order=2, channels=8, seq_len=T, masked=False, seed=T)
    opts = dict(top_k=(4, 8), mass_aware=mass_aware)
    assert_pairs(f"T={T}", run_gpu(case, **opts), run_oracle(case, dense=True, **opts), None, FP32_TOL)


@pytest.mark.parametrize("mass_aware", [False, True], ids=["plain", "mass_aware"])
@pytest.mark.parametrize("re_norm", TOP_K_RE_NORM_SETTINGS, ids=lambda r: "r{}-{}".format(*r))
@pytest.mark.parametrize("shape", SHAPE_CASES, ids=lambda s: "U{}P{}C{}T{}".format(*s))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_low_precision_parallel(dtype, shape, re_norm, mass_aware):
    """test_ram_attention_numerics.py:68-87, against the fp64 oracle on the
    quantised inputs (the reference compares with its own fp32 run of them)."""
    U, P, C, T = shape
    print(f"grid {dtype} U={U} P={P} C={C} T={T} re_norm={re_norm} mass_aware={mass_aware}", flush=True)
    case = cast_case(make_ram_case(order=U, radix=P, channels=C, seq_len=T, seed=sum(shape) + 1), dtype)
    opts = dict(re_norm=re_norm, mass_aware=mass_aware)
    assert_pairs(str(dtype), run_gpu(case, **opts), run_oracle(case, **opts), case.mask, LOW_TOL)


@pytest.mark.parametrize("mass_aware", [False, True], ids=["plain", "mass_aware"])
@pytest.mark.parametrize("re_norm", TOP_K_RE_NORM_SETTINGS, ids=lambda r: "r{}-{}".format(*r))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_low_precision_autoregressive(dtype, re_norm, mass_aware):
    """test_ram_attention_numerics.py:89-105: single-token decode steps
    (chunks of one token, no gradients) from a masked sequence."""
    case = cast_case(make_ram_case(order=3, channels=16, seq_len=33, seed=33), dtype)
    opts = dict(re_norm=re_norm, mass_aware=mass_aware)
    got = run_gpu(case, chunk=1, grad=False, **opts)
    assert_pairs(f"{dtype} decode", got, run_oracle(case, grad=False, **opts), case.mask, LOW_TOL)


@pytest.mark.parametrize("mass_aware", [False, True], ids=["plain", "mass_aware"])
@pytest.mark.parametrize("op", ["ram_attn_forward_", "topk_segment_forward_", "api_inplace"])
def test_inplace_forms_match_dense_oracle(op, mass_aware):
    """The in-place prefill (reference topk_segment_forward_,
    ram_attn_ops.cpp:312-347) from a random non-zero state with a mask,
    T > 1, against the dense fp64 restatement; the state tensors passed in
    are the ones updated."""
    case = make_ram_case(order=3, radix=5, channels=24, seq_len=97, seed=97)
    B, H, U, P, T = case.w_addr.shape
    A = P ** U
    re_norm = (0.25, 0.75)
    print(f"in-place {op} mass_aware={mass_aware}", flush=True)
    slot, mass = case.init_slot.to(DEV).clone(), case.init_mass.to(DEV).clone()
    d = {k: getattr(case, k).to(DEV) for k in ("w_addr", "r_addr", "values", "gamma", "position_ids", "mask")}
    ops = torch.ops.ramnet_ops
    if op == "ram_attn_forward_":
        y = ops.ram_attn_forward_(d["w_addr"], d["r_addr"], d["values"], d["gamma"], slot, mass, d["mask"],
                                  EMBED_NUM, d["position_ids"], 8, 8, *re_norm, mass_aware, EPS)
    elif op == "topk_segment_forward_":
        idx, val = ops.topk_addr_forward(d["w_addr"], d["r_addr"], EMBED_NUM, A, d["position_ids"], 8, 8, *re_norm)
        y = ops.topk_segment_forward_(idx, val, d["values"], d["gamma"], slot, mass, d["mask"], 8, 8, mass_aware,
                                      EPS)
    else:
        from ramnet_ops import random_access_memory_attention as ram
        y, (s2, m2) = ram(d["w_addr"].permute(0, 4, 1, 2, 3), d["r_addr"].permute(0, 4, 1, 2, 3),
                          d["values"].permute(0, 2, 1, 3), d["gamma"].permute(0, 2, 1), init_ram=(slot, mass),
                          mask=d["mask"], embed_num=EMBED_NUM, position_ids=d["position_ids"], top_k=8,
                          top_k_re_norm=re_norm, mass_aware=mass_aware, inplace=True)
        assert s2.data_ptr() == slot.data_ptr() and m2.data_ptr() == mass.data_ptr()
        y = y.permute(0, 2, 1, 3)
    torch.cuda.synchronize()
    got = ((y.cpu(), slot.cpu(), mass.cpu()), None)
    ref = run_oracle(case, re_norm=re_norm, mass_aware=mass_aware, grad=False, dense=True)
    assert not torch.equal(got[0][1], case.init_slot), "the state was not updated in place"
    assert_pairs(op, got, ref, case.mask, FP32_TOL)


@pytest.mark.parametrize("top_k", TOP_K_SETTINGS, ids=lambda k: "K{}-{}".format(*k))
def test_autoregressive_matches_parallel(top_k):
    """Single-token decode steps (the fused decode op, one call per token,
    state carried in place) == one parallel call, and == the fp64 event loop
    on the decoder's selection, over the reference's top-K range at A = 1024
    (order 5, radix 4), every re-norm setting and mass_aware, without and
    with per-row masks (reference test_ram_attention_behavior.py:90-109).
    fp32 rel <= 1e-5; masked tokens read exactly 0 in both paths."""
    case = make_ram_case(batch=3, heads=4, order=5, channels=16, seq_len=65, masked=False, seed=31)
    mask = torch.ones(3, 65, dtype=torch.bool)
    mask[0, ::3] = False
    mask[1, 1::4] = False
    mask[2, 2::5] = False
    mask[:, 7::16] = False
    positions = (mask.long().cumsum(-1) - 1).masked_fill(~mask, 0)
    masked = replace(case, mask=mask, position_ids=positions)
    for re_norm in TOP_K_RE_NORM_SETTINGS:
        for mass_aware in (False, True):
            for name, inputs in (("plain", case), ("masked", masked)):
                label = f"AR == PARALLEL top_k={top_k} re_norm={re_norm} mass_aware={mass_aware} {name}"
                print(label, flush=True)
                ar, _ = run_gpu(inputs, top_k=top_k, re_norm=re_norm, mass_aware=mass_aware, chunk=1, grad=False)
                par, _ = run_gpu(inputs, top_k=top_k, re_norm=re_norm, mass_aware=mass_aware, grad=False)
                ref, _ = run_oracle(inputs, top_k=top_k, re_norm=re_norm, mass_aware=mass_aware, grad=False)
                for what, other in (("parallel", par), ("fp64 event loop", ref)):
                    for tname, a, b in zip(("y", "slot", "mass"), ar, other):
                        err = oracle.rel_err(a, b)
                        assert err <= FP32_TOL, f"{label}: {tname} vs {what} rel err {err:.3e}"
                if inputs.mask is not None:
                    off = ~inputs.mask[:, None, :, None].expand_as(ar[0])
                    assert bool((ar[0][off] == 0).all()), f"{label}: masked tokens must read 0"

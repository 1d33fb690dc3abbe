"""The multi-step decode entry point (``ramnet_topk_autoregressive_steps_``).

* S steps in one call equal S calls of the single-step op on the step slices
  of the inputs, bit for bit (y, slot and mass): the persistent kernel runs
  the single-step kernel's stages in a software-pipelined loop, and shapes
  outside its envelope run one single-step launch per step. The cases cover
  both kernels' template forms (top-k up to 8 and up to 11, two and four
  channels per lane, full and partial channel counts), all three dtypes,
  mass_aware, re-normalisation, CAPE, per-(step, batch) masks, a slot that
  is written on consecutive steps, and the per-step fallback (top-k 16,
  P = 64).
* At the config-3 shape (B=64, H=16, the 64x16x1024x128 state), 16 steps in
  one launch against the stepwise fp64 event loop of the oracle: every
  step's y and the final state of several (b, h) heads.

Bars: bit-equal to the single-step op; against the oracle fp32 state
rel <= 1e-5 and bf16 y rel <= 2e-2 (max|a-b| / max|b|).
"""
from __future__ import annotations

import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
LOW_TOL = 2e-2
DEV = "cuda"


def _ops():
    import ramnet_ops  # noqa: F401  (registers torch.ops.ramnet_ops.*)
    from ramnet_ops import _native
    _native.lib()
    return torch.ops.ramnet_ops


def _inputs(S, B, H, U, P, C, dtype, seed, masked=False, repeat=False):
    A = P ** U
    g = torch.Generator(device=DEV).manual_seed(seed)
    lg = torch.randn(S, 2, B, H, U, P, device=DEV, generator=g) * 2.0
    if repeat:  # the same write address on steps 1 and 2: a slot written on consecutive steps
        lg[2, 0] = lg[1, 0]
    w, r = lg[:, 0].to(dtype).contiguous(), lg[:, 1].to(dtype).contiguous()
    x = torch.randn(S, B, H, C, device=DEV, generator=g).to(dtype)
    gamma = torch.randn(S, B, H, device=DEV, generator=g).to(dtype)
    pos = torch.randint(0, 3 * A, (S, B), device=DEV, generator=g).to(torch.int32)
    mask = (torch.rand(S, B, device=DEV, generator=g) > 0.3) if masked else torch.empty(0, dtype=torch.bool,
                                                                                        device=DEV)
    slot = 0.5 * torch.randn(B, H, A, C, device=DEV, generator=g)
    mass = torch.rand(B, H, A, device=DEV, generator=g) + 0.01
    return w, r, x, gamma, pos, mask, slot, mass


CASES = [
    # S, B, H, U, P, C, K, dtype, mass_aware, re_norm, masked, repeat
    (9, 4, 4, 2, 32, 128, 8, torch.bfloat16, False, 0.0, False, True),     # the config-3 kernel form
    (7, 3, 4, 2, 16, 100, 4, torch.float32, True, 0.0, True, True),        # partial channels, masks
    (6, 2, 3, 3, 8, 256, 11, torch.float16, False, 0.5, True, False),     # top-k <= 11 form, 4 channels/lane
    (5, 2, 4, 2, 32, 64, 8, torch.float32, True, 1.0, False, True),        # C = 64
    (1, 3, 2, 2, 32, 128, 8, torch.bfloat16, False, 0.0, True, False),     # one step
    (4, 2, 4, 2, 32, 128, 16, torch.bfloat16, False, 0.0, True, True),     # per-step fallback: top-k 16
    (4, 2, 2, 2, 64, 96, 8, torch.float32, False, 0.0, False, False),      # per-step fallback: P = 64
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"S{c[0]}B{c[1]}H{c[2]}U{c[3]}P{c[4]}C{c[5]}K{c[6]}"
                                                     f"{str(c[7])[6:]}{'-ma' if c[8] else ''}"
                                                     f"{'-rn' if c[9] else ''}{'-mask' if c[10] else ''}")
def test_steps_equal_single_steps(case):
    ops = _ops()
    S, B, H, U, P, C, K, dtype, mass_aware, re_norm, masked, repeat = case
    E = H // 2
    print(f"decode steps vs single steps: {case}", flush=True)
    w, r, x, gamma, pos, mask, slot0, mass0 = _inputs(S, B, H, U, P, C, dtype, seed=11, masked=masked, repeat=repeat)
    slot_a, mass_a = slot0.clone(), mass0.clone()
    ys = []
    for s in range(S):
        ms = mask[s] if masked else mask
        ys.append(ops.topk_autoregressive_(w[s], r[s], x[s], gamma[s], slot_a, mass_a, ms, E, pos[s], K, K, re_norm,
                                           re_norm, mass_aware, 1e-12))
    y_a = torch.stack(ys)
    slot_b, mass_b = slot0.clone(), mass0.clone()
    y_b = ops.topk_autoregressive_steps_(w, r, x, gamma, slot_b, mass_b, mask, E, pos, K, K, re_norm, re_norm,
                                         mass_aware, 1e-12)
    torch.cuda.synchronize()
    assert y_b.shape == y_a.shape and y_b.dtype == y_a.dtype
    assert torch.equal(y_a, y_b), f"y differs: max {(y_a.float() - y_b.float()).abs().max().item():.3e}"
    assert torch.equal(slot_a, slot_b), "slot state differs"
    assert torch.equal(mass_a, mass_b), "mass state differs"
    assert not torch.equal(slot_a, slot0), "the steps wrote nothing"
    if masked:
        assert (y_b[~mask] == 0).all(), "masked steps must give y = 0"


def test_steps_zero_steps_is_a_no_op():
    ops = _ops()
    w, r, x, gamma, pos, mask, slot, mass = _inputs(1, 2, 2, 2, 16, 64, torch.float32, seed=2)
    s0, m0 = slot.clone(), mass.clone()
    y = ops.topk_autoregressive_steps_(w[:0], r[:0], x[:0], gamma[:0], slot, mass, mask, 1, pos[:0], 4, 4, 0.0, 0.0,
                                       False, 1e-12)
    torch.cuda.synchronize()
    assert y.shape == (0, 2, 2, 64)
    assert torch.equal(slot, s0) and torch.equal(mass, m0)


def test_config3_persistent_steps_match_oracle():
    """Config 3 (B=64, H=16, 1024 slots of 128 channels per head, K=8, bf16)
    as the benchmark's persistent line runs it: 16 steps in one launch."""
    ops = _ops()
    B, H, C, U, P, K, S = 64, 16, 128, 2, 32, 8, 16
    A = P ** U
    E = H // 2
    print(f"config 3: {S} steps in one launch at B={B}, H={H}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(4)
    slot = 0.5 * torch.randn(B, H, A, C, device=DEV, generator=g)
    mass = torch.full((B, H, A), 1.0 / A, device=DEV)
    d_k = 128
    W = torch.randn(H, d_k, U * P, device=DEV, generator=g) / d_k ** 0.5
    q = torch.randn(S, 2, B, H, d_k, device=DEV, generator=g)
    lg = (torch.einsum('sqbhd,hdn->sqbhn', q, W) / U ** 0.5).to(torch.bfloat16).view(S, 2, B, H, U, P)
    w_all, r_all = lg[:, 0].contiguous(), lg[:, 1].contiguous()
    x_all = torch.randn(S, B, H, C, device=DEV, generator=g).to(torch.bfloat16)
    g_all = torch.sigmoid(torch.randn(S, B, H, device=DEV, generator=g)).to(torch.bfloat16)
    t0 = torch.randint(0, 8192, (B,), device=DEV, generator=g)
    pos_all = (t0.view(1, B) + torch.arange(S, device=DEV).view(S, 1)).to(torch.int32).contiguous()
    no_mask = torch.empty(0, dtype=torch.bool, device=DEV)

    heads = ((0, 0), (17, 5), (33, 8), (63, 15), (40, 12))
    sel = lambda t: torch.stack([t[b, h] for b, h in heads]).unsqueeze(1).cpu()  # (n, 1, ...)
    slot_before, mass_before = sel(slot), sel(mass)
    y = ops.topk_autoregressive_steps_(w_all, r_all, x_all, g_all, slot, mass, no_mask, E, pos_all, K, K, 0.0, 0.0,
                                       False, 1e-12)
    torch.cuda.synchronize()
    slot_after, mass_after = sel(slot), sel(mass)

    wi, wv, ri, rv = [], [], [], []
    for s in range(S):
        for lgs, ii, vv in ((w_all[s], wi, wv), (r_all[s], ri, rv)):
            idx, val = ops.topk_addr_single_forward(lgs.unsqueeze(-1), E, A, pos_all[s].view(B, 1), K, 0.0, False,
                                                    False)
            oracle.check_topk_indices(idx.cpu(), lgs.unsqueeze(-1).cpu(), E, pos_all[s].view(B, 1).cpu().long(), K,
                                      encode_batch_idx=False)
            local = idx.cpu() - (torch.arange(H) * A).view(1, H, 1, 1)
            ii.append(sel(local)[..., 0])
            vv.append(sel(val)[..., 0])
    stack = lambda lst: torch.stack(lst, dim=-1)  # (n, 1, K, S)
    xs = torch.stack([sel(x_all[s]) for s in range(S)], dim=2).double()  # (n, 1, S, C)
    gs = torch.stack([sel(g_all[s]) for s in range(S)], dim=-1).double()  # (n, 1, S)
    ry, rslot, rmass = oracle.sparse_gsu_f64(stack(wi), stack(wv), stack(ri), stack(rv), xs, gs, slot_before,
                                             mass_before, None, False, 1e-12, encoded=False)
    ry = torch.as_tensor(ry)
    y_sel = torch.stack([sel(y[s]) for s in range(S)], dim=2)  # (n, 1, S, C)
    for s in range(S):
        err = oracle.rel_err(y_sel[:, :, s], ry[:, :, s])
        assert err <= LOW_TOL, f"y of step {s}: rel err {err:.3e}"
    assert oracle.rel_err(slot_after, rslot) <= FP32_TOL, "slot state after the steps"
    assert oracle.rel_err(mass_after, rmass) <= FP32_TOL, "mass state after the steps"

"""Argument checks of the registered operators called directly.

Every ``torch.ops.ramnet_ops.*`` operator takes its sizes from one or two
tensors and indexes all the others with them, so each tensor argument is
checked against those sizes before anything is launched, as the
reference's native checks do (check_tensor, csrc/cuda_utils.cuh:375-391,
ram_attn_topk_autoregressive.cu:216-224): a mis-shaped tensor raises
RuntimeError. The tensors live on the GPU (the operators refuse host
tensors first), but every call below fails on the host.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
B, H, U, P, T, C, K = 2, 3, 2, 4, 9, 8, 4
A = P ** U


def _ops():
    import ramnet_ops  # noqa: F401
    return torch.ops.ramnet_ops


def _t(*shape, dtype=torch.float32):
    return torch.zeros(*shape, dtype=dtype, device=DEV)


def _raises(fn, *args):
    with pytest.raises(RuntimeError, match="shape mismatch|dimensions|must equal P"):
        fn(*args)


def test_decoder_ops_reject_mis_shaped_tensors():
    ops = _ops()
    addr = _t(B, H, U, P, T)
    pos = _t(B, T, dtype=torch.int32)
    _raises(ops.topk_addr_single_forward, _t(B, H, U, P), 0, A, pos, K, 0.0, False, True)
    _raises(ops.topk_addr_single_forward, addr, 0, A, _t(B, T + 1, dtype=torch.int32), K, 0.0, False, True)
    _raises(ops.topk_addr_single_forward, addr, 0, A + 1, pos, K, 0.0, False, True)
    _raises(ops.topk_addr_forward, addr, _t(B, H, U, P, T - 1), 0, A, pos, K, K, 0.0, 0.0)
    _raises(ops.topk_addr_forward, addr, addr, 0, A, _t(B + 1, T, dtype=torch.int32), K, K, 0.0, 0.0)
    ev = _t(B, H, 2 * K, T)
    idx = _t(B, H, 2 * K, T, dtype=torch.int32)
    shape = [B, H, U, P, A, T]
    _raises(ops.topk_addr_backward, idx, ev, addr, addr, _t(B, H, 2 * K, T - 1), 0, pos, K, K, 0.0, 0.0, shape,
            torch.float32)
    _raises(ops.topk_addr_backward, idx, _t(B, H, 2 * K + 1, T), addr, addr, ev, 0, pos, K, K, 0.0, 0.0, shape,
            torch.float32)
    _raises(ops.topk_addr_single_backward, idx[:, :, :K], ev[:, :, :K], _t(B, H, U, P + 1, T), ev[:, :, :K], 0, pos,
            K, 0.0, False, shape, torch.float32)


def test_segment_ops_reject_mis_shaped_tensors():
    ops = _ops()
    idx = _t(B, H, 2 * K, T, dtype=torch.int32)
    val = _t(B, H, 2 * K, T)
    x, gamma = _t(B, H, T, C), _t(B, H, T)
    slot, mass = _t(B, H, A, C), _t(B, H, A)
    mask = torch.ones(B, T, dtype=torch.bool, device=DEV)
    good = dict(idx=idx, val=val, x=x, gamma=gamma, slot=slot, mass=mass, mask=mask)
    bad = dict(idx=_t(B, H, 2 * K, T + 1, dtype=torch.int32), val=_t(B, H, K, T), x=_t(B, H, T, C, 1),
               gamma=_t(B, H, T + 2), slot=_t(B - 1, H, A, C), mass=_t(B, H, A + 1),
               mask=torch.ones(B, T - 1, dtype=torch.bool, device=DEV))
    for name in good:
        a = {**good, name: bad[name]}
        _raises(ops.topk_segment_forward, a["idx"], a["val"], a["x"], a["gamma"], a["slot"], a["mass"], a["mask"], K,
                K, False, 1e-12)
        _raises(ops.topk_segment_forward_, a["idx"], a["val"], a["x"], a["gamma"], a["slot"].clone(),
                a["mass"].clone(), a["mask"], K, K, False, 1e-12)
        _raises(ops.topk_segment_backward, a["idx"], a["val"], a["x"], a["gamma"], a["slot"], a["mass"], a["mask"],
                x, None, None, K, K, False, 1e-12)
    _raises(ops.topk_segment_backward, idx, val, x, gamma, slot, mass, mask, _t(B, H, T, C + 1), None, None, K, K,
            False, 1e-12)
    _raises(ops.topk_segment_backward, idx, val, x, gamma, slot, mass, mask, x, _t(B, H, A, C + 1), None, K, K,
            False, 1e-12)


def test_fused_and_decode_ops_reject_mis_shaped_tensors():
    ops = _ops()
    w = _t(B, H, U, P, T)
    x, gamma = _t(B, H, T, C), _t(B, H, T)
    slot, mass = _t(B, H, A, C), _t(B, H, A)
    pos = _t(B, T, dtype=torch.int32)
    for args in ((w, w, x, gamma, _t(B, H, A * 2, C), mass), (w, w, x, gamma, slot, _t(B, H)),
                 (w, w, _t(B, H, T - 1, C), gamma, slot, mass), (w, _t(B, H, U, P, T + 1), x, gamma, slot, mass)):
        _raises(ops.ram_attn_forward, *args, None, 0, pos, K, K, 0.0, 0.0, False, 1e-12)
        _raises(ops.ram_attn_forward_, *args, None, 0, pos, K, K, 0.0, 0.0, False, 1e-12)
    _raises(ops.ram_attn_forward, w, w, x, gamma, slot, mass, None, 0, _t(B, T + 3, dtype=torch.int32), K, K, 0.0,
            0.0, False, 1e-12)
    wd, xd, gd = _t(B, H, U, P), _t(B, H, C), _t(B, H)
    pd = _t(B, dtype=torch.int32)
    empty = torch.empty(0, dtype=torch.bool, device=DEV)
    for args in ((wd, wd, xd, gd, slot, _t(B, H, A - 1), empty, pd),
                 (wd, wd, xd, gd, _t(B + 1, H, A, C), _t(B + 1, H, A), empty, pd),
                 (wd, _t(B, H, U, P + 1), xd, gd, slot, mass, empty, pd),
                 (wd, wd, _t(B, H, C + 4), gd, slot, mass, empty, pd),
                 (wd, wd, xd, _t(B, H, 1), slot, mass, empty, pd),
                 (wd, wd, xd, gd, slot, mass, torch.ones(B + 1, dtype=torch.bool, device=DEV), pd),
                 (wd, wd, xd, gd, slot, mass, empty, _t(B, 1, dtype=torch.int32)),
                 (_t(B, H, U, P + 1), _t(B, H, U, P + 1), xd, gd, slot, mass, empty, pd)):
        w_, r_, x_, g_, s_, m_, mk, p_ = args
        _raises(ops.topk_autoregressive_, w_, r_, x_, g_, s_.clone(), m_.clone(), mk, 0, p_, K, K, 0.0, 0.0, False,
                1e-12)


def test_decode_ops_reject_logits_of_another_dtype():
    """The decode kernels read the logits in x's dtype: bf16 or fp16 logits
    with fp32 values (or the other way round) raise RuntimeError before any
    launch, as the reference's check_address does
    (ram_attn_topk_autoregressive.cu:32-34,216)."""
    ops = _ops()
    S = 3
    slot, mass = _t(B, H, A, C), _t(B, H, A)
    empty = torch.empty(0, dtype=torch.bool, device=DEV)
    for xd, ld in ((torch.float32, torch.bfloat16), (torch.float32, torch.float16), (torch.bfloat16, torch.float32)):
        x, g = _t(B, H, C, dtype=xd), _t(B, H, dtype=xd)
        good, bad = _t(B, H, U, P, dtype=xd), _t(B, H, U, P, dtype=ld)
        pd = _t(B, dtype=torch.int32)
        for w_, r_ in ((bad, good), (good, bad), (bad, bad)):
            with pytest.raises(RuntimeError, match="dtype mismatch"):
                ops.topk_autoregressive_(w_, r_, x, g, slot.clone(), mass.clone(), empty, 0, pd, K, K, 0.0, 0.0,
                                         False, 1e-12)
        xs, gs = _t(S, B, H, C, dtype=xd), _t(S, B, H, dtype=xd)
        gs_, bs_ = _t(S, B, H, U, P, dtype=xd), _t(S, B, H, U, P, dtype=ld)
        ps = _t(S, B, dtype=torch.int32)
        for w_, r_ in ((bs_, gs_), (gs_, bs_)):
            with pytest.raises(RuntimeError, match="dtype mismatch"):
                ops.topk_autoregressive_steps_(w_, r_, xs, gs, slot.clone(), mass.clone(), empty, 0, ps, K, K, 0.0,
                                               0.0, False, 1e-12)

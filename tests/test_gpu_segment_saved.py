"""The training pair with saved rows (topk_segment_forward_saved +
topk_segment_backward_saved) on the GPU.

The forward keeps, per event, x - s before each write and the row of each
read; the backward then runs one pass over the sequence. The pair has no
counterpart in the reference (whose backward reconstructs the forward,
csrc/ram_attn_segment_parallel.cu:418-606), so its contract is that of
topk_segment_forward / topk_segment_backward on the same inputs: gradients
against fp64 autograd of the dense oracle at the backward tests' bar, and
against the recompute pair to fp32 rounding (the read dot products are
summed in another order).
"""
from __future__ import annotations

import pytest
import torch

import oracle
from test_gpu_segment_backward import _check, _inputs, _oracle, _tol

pytestmark = pytest.mark.gpu

DEV = "cuda"
F32, BF16, F16 = torch.float32, torch.bfloat16, torch.float16

CASES = [
    # B, H, U, P, T, C, Kw, Kr, dtype, masked, mass_aware: shapes the pair takes
    (2, 2, 2, 8, 40, 16, 4, 4, F32, False, False),
    (2, 2, 3, 4, 29, 32, 8, 8, F32, True, True),      # mass_aware, masked tokens, a ragged last chunk
    (1, 2, 2, 8, 21, 16, 40, 24, F32, False, True),   # 64 event lanes: one channel per backward slice
    (1, 2, 2, 16, 1, 16, 8, 8, F32, False, True),     # T = 1
    (2, 2, 2, 16, 40, 64, 16, 16, BF16, True, False),  # 16 events: 16-event forward lanes
    (1, 2, 2, 16, 40, 64, 8, 8, F16, False, True),
    (1, 2, 2, 4, 45, 16, 8, 8, F32, False, False),    # A = 16: neighbouring tokens share slots
    (1, 3, 2, 16, 70, 128, 8, 8, BF16, True, True),   # config-2 lanes (32-channel forward slices)
]


def _ops():
    import ramnet_ops  # noqa: F401
    return torch.ops.ramnet_ops


def _nat():
    from ramnet_ops import _native
    return _native


def _id(c):
    return "-".join(str(v).replace("torch.", "") for v in c)


@pytest.mark.parametrize("case", CASES, ids=_id)
def test_saved_pair_matches_oracle_and_recompute(case):
    B, H, U, P, T, C, Kw, Kr, dtype, masked, mass_aware = case
    ops, nat = _ops(), _nat()
    print(f"saved pair case {case}", flush=True)
    d = _inputs(B, H, U, P, T, C, Kw, Kr, dtype, masked, seed=B * 1000 + T * 10 + C + Kw + 3)
    A = d["A"]
    assert nat.segment_saved_bytes(B, H, T, A, C, Kw, Kr, dtype) > 0, "the case must take the saved pair"
    idx, val = ops.topk_addr_forward(d["w"].to(DEV), d["r"].to(DEV), 1, A, d["pos"].to(DEV).int(), Kw, Kr, 0.0, 0.0)
    mask = None if d["mask"] is None else d["mask"].to(DEV)
    x, gamma, slot, mass = d["x"].to(DEV), d["gamma"].to(DEV), d["slot"].to(DEV), d["mass"].to(DEV)
    Dy, Ds, Dm = d["Dy"].to(DEV), d["Ds"].to(DEV), d["Dm"].to(DEV)

    y, s, m, saved = ops.topk_segment_forward_saved(idx, val, x, gamma, slot, mass, mask, Kw, Kr, mass_aware, 1e-12)
    y0, s0, m0 = ops.topk_segment_forward(idx, val, x, gamma, slot, mass, mask, Kw, Kr, mass_aware, 1e-12)
    got = ops.topk_segment_backward_saved(val, x, gamma, slot, mass, saved, Dy, Ds, Dm, Kw, Kr, mass_aware, 1e-12)
    rec = ops.topk_segment_backward(idx, val, x, gamma, slot, mass, mask, Dy, Ds, Dm, Kw, Kr, mass_aware, 1e-12)
    torch.cuda.synchronize()

    # forward outputs: those of topk_segment_forward (its layout may differ,
    # so y may differ in the order of its read sum)
    keep = torch.ones(B, T, dtype=torch.bool) if d["mask"] is None else d["mask"]
    for name, a, b in (("y", y.cpu()[keep[:, None].expand(B, H, T)], y0.cpu()[keep[:, None].expand(B, H, T)]),
                       ("slot", s.cpu(), s0.cpu()), ("mass", m.cpu(), m0.cpu())):
        err = oracle.rel_err(a.double(), b.double())
        print(f"  forward {name}: rel {err:.2e} vs topk_segment_forward", flush=True)
        assert err <= (1e-6 if dtype == F32 or name != "y" else 1e-2), name
    # gradients: fp64 autograd of the dense oracle, and the recompute pair
    ref = _oracle(idx.cpu(), val.cpu(), d["x"], d["gamma"], d["slot"], d["mass"], d["mask"], d["Dy"], d["Ds"],
                  d["Dm"], Kw, Kr, mass_aware, 1e-12, U, P)
    names = ("D_addr_val", "D_x", "D_gamma", "D_slot", "D_mass")
    for name, g, r in zip(names, got, ref):
        _check(name, g, r, _tol(dtype))
    for name, g, r in zip(names, got, rec):
        err = oracle.rel_err(g.cpu().double(), r.cpu().double())
        print(f"  {name}: rel {err:.2e} vs topk_segment_backward", flush=True)
        assert err <= 1e-6, name
    # the saved buffer is only read: a second backward gives the same bits
    again = ops.topk_segment_backward_saved(val, x, gamma, slot, mass, saved, Dy, Ds, Dm, Kw, Kr, mass_aware, 1e-12)
    for a, b in zip(got, again):
        assert torch.equal(a, b)


def test_saved_pair_shape_envelope():
    """Shapes outside the pair's envelope report -1 (the API then runs the
    recompute pair), and the ops refuse them with RuntimeError."""
    ops, nat = _ops(), _nat()
    # C = 24 is no multiple of a 16- or 32-channel forward slice at top-k 8
    assert nat.segment_saved_bytes(1, 2, 16, 64, 24, 8, 8, F32) == -1
    assert nat.segment_saved_bytes(1, 2, 16, 64, 32, 8, 8, F32) > 0
    # two passes of events (top-k above 64), and T = 0
    assert nat.segment_saved_bytes(1, 1, 13, 256, 16, 100, 70, F32) == -1
    assert nat.segment_saved_bytes(1, 1, 0, 64, 32, 8, 8, F32) == -1
    B, H, T, A, C, K = 1, 2, 16, 64, 24, 8
    idx = torch.zeros(B, H, 2 * K, T, dtype=torch.int32, device=DEV)
    val = torch.zeros(B, H, 2 * K, T, device=DEV)
    x = torch.zeros(B, H, T, C, device=DEV)
    with pytest.raises(RuntimeError, match="saved-row"):
        ops.topk_segment_forward_saved(idx, val, x, torch.zeros(B, H, T, device=DEV),
                                       torch.zeros(B, H, A, C, device=DEV), torch.ones(B, H, A, device=DEV), None, K,
                                       K, False, 1e-12)


@pytest.mark.parametrize("mass_aware", [False, True])
def test_api_gradients_through_saved_pair(mass_aware):
    """random_access_memory_attention with grad at a shape the saved pair
    takes: its gradients equal those of the recompute pair's composition."""
    from ramnet_ops import random_access_memory_attention
    ops, nat = _ops(), _nat()
    B, H, U, P, T, C, K, E = 2, 3, 2, 8, 50, 32, 6, 2
    A = P ** U
    assert nat.segment_saved_bytes(B, H, T, A, C, K, K, BF16) > 0
    d = _inputs(B, H, U, P, T, C, K, K, BF16, True, seed=31 + int(mass_aware))
    print(f"api gradients through the saved pair, mass_aware={mass_aware}", flush=True)

    def run(composition):
        leaves = {k: d[k].to(DEV).requires_grad_(True) for k in ("w", "r", "x", "gamma", "slot", "mass")}
        mask = d["mask"].to(DEV)
        if composition:
            y, (slot, mass) = random_access_memory_attention(
                leaves["w"].permute(0, 4, 1, 2, 3), leaves["r"].permute(0, 4, 1, 2, 3), leaves["x"].permute(0, 2, 1, 3),
                leaves["gamma"].permute(0, 2, 1), init_ram=(leaves["slot"], leaves["mass"]), mask=mask, embed_num=E,
                position_ids=d["pos"].to(DEV), top_k=K, mass_aware=mass_aware)
            y = y.permute(0, 2, 1, 3)
        else:
            idx, val = ops.topk_addr_forward(leaves["w"], leaves["r"], E, A, d["pos"].to(DEV).int(), K, K, 0.0, 0.0)
            y, slot, mass = ops.topk_segment_forward(idx, val, leaves["x"], leaves["gamma"], leaves["slot"],
                                                     leaves["mass"], mask, K, K, mass_aware, 1e-12)
        loss = (y.float() * d["Dy"].float().to(DEV)).sum() + (slot * d["Ds"].to(DEV)).sum() \
            + (mass * d["Dm"].to(DEV)).sum()
        loss.backward()
        return {k: v.grad.cpu().double() for k, v in leaves.items()}

    a, b = run(True), run(False)
    for k in a:
        err = oracle.rel_err(a[k], b[k])
        print(f"  {k}: rel {err:.2e}", flush=True)
        assert err <= 1e-5, k


def test_config2_full_size_saved_pair_heads():
    """Config 2 at full size through the saved pair (the training step's
    path): two heads against the fp64 state-reconstruction oracle."""
    from ram_cases import projected_logits
    ops, nat = _ops(), _nat()
    B, H, U, P, T, C, K = 8, 16, 2, 32, 4096, 128, 8
    A = P ** U
    assert nat.segment_saved_bytes(B, H, T, A, C, K, K, BF16) > 0
    print("config 2 full-size saved pair", flush=True)
    w, r = projected_logits(B, H, U, P, T, 128, seed=2)
    g = torch.Generator().manual_seed(23)
    x = torch.randn(B, H, T, C, generator=g).to(torch.bfloat16)
    gamma = torch.sigmoid(torch.randn(B, H, T, generator=g) - 1).to(torch.bfloat16)
    pos = torch.arange(T).view(1, T).expand(B, T)
    Dy = torch.randn(B, H, T, C, generator=g).to(torch.bfloat16)
    slot0 = torch.zeros(B, H, A, C)
    mass0 = torch.full((B, H, A), 1.0 / A)
    idx, val = ops.topk_addr_forward(w.to(DEV), r.to(DEV), H // 2, A, pos.to(DEV), K, K, 0.0, 0.0)
    _, _, _, saved = ops.topk_segment_forward_saved(idx, val, x.to(DEV), gamma.to(DEV), slot0.to(DEV), mass0.to(DEV),
                                                    None, K, K, False, 1e-12)
    got = ops.topk_segment_backward_saved(val, x.to(DEV), gamma.to(DEV), slot0.to(DEV), mass0.to(DEV), saved,
                                          Dy.to(DEV), None, None, K, K, False, 1e-12)
    torch.cuda.synchronize()
    del saved
    got = [t.cpu() for t in got]
    idx_c, val_c = idx.cpu(), val.cpu()
    heads = ((0, 0), (7, 15))
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


def test_config4_full_size_saved_pair_heads():
    """Config 4 at full size through the saved pair (B=4, H=8, T=8192, U=3,
    P=16 -> A=4096, K=16, bf16): the 16-event saving scan and the saved
    backward with two channels per lane, two heads against the fp64
    state-reconstruction oracle."""
    from ram_cases import projected_logits
    ops, nat = _ops(), _nat()
    B, H, U, P, T, C, K, E = 4, 8, 3, 16, 8192, 128, 16, 4
    A = P ** U
    assert nat.segment_saved_bytes(B, H, T, A, C, K, K, BF16) > 0
    print("config 4 full-size saved pair", flush=True)
    w, r = projected_logits(B, H, U, P, T, 128, seed=4, dtype=torch.float32)
    w, r = w.to(torch.bfloat16), r.to(torch.bfloat16)
    g = torch.Generator().manual_seed(43)
    x = torch.randn(B, H, T, C, generator=g).to(torch.bfloat16)
    gamma = torch.sigmoid(torch.randn(B, H, T, generator=g)).to(torch.bfloat16)
    pos = torch.arange(T).view(1, T).expand(B, T)
    Dy = torch.randn(B, H, T, C, generator=g).to(torch.bfloat16)
    slot0 = torch.zeros(B, H, A, C)
    mass0 = torch.full((B, H, A), 1.0 / A)
    idx, val = ops.topk_addr_forward(w.to(DEV), r.to(DEV), E, A, pos.to(DEV), K, K, 0.0, 0.0)
    _, _, _, saved = ops.topk_segment_forward_saved(idx, val, x.to(DEV), gamma.to(DEV), slot0.to(DEV), mass0.to(DEV),
                                                    None, K, K, False, 1e-12)
    got = ops.topk_segment_backward_saved(val, x.to(DEV), gamma.to(DEV), slot0.to(DEV), mass0.to(DEV), saved,
                                          Dy.to(DEV), None, None, K, K, False, 1e-12)
    torch.cuda.synchronize()
    del saved
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

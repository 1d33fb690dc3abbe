"""Pin the CPU oracle before trusting it (CPU only).

Each oracle function is checked against something it does not compute
itself: the reference tests' known-answer fixtures (tests/golden/), closed
forms of the mathematics, a pure-Python brute force on tiny inputs, and the
other oracle algorithm (dense fp32 torch vs sparse fp64 event loop).
"""
from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch

import oracle
from ram_cases import make_case


def _dense_map(idx, val, A, H, encode=True):
    idx = torch.as_tensor(idx).long()
    B, _, K, T = idx.shape
    base = (torch.arange(B * H).view(B, H, 1, 1) if encode else torch.arange(H).view(1, H, 1, 1)) * A
    out = torch.zeros(B, H, T, A, dtype=torch.float64)
    out.scatter_(-1, (idx - base).permute(0, 1, 3, 2), torch.as_tensor(val).double().permute(0, 1, 3, 2))
    return out


# ---------------------------------------------------------------------------
# decoder

@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-12), (torch.float32, 1e-6)])
def test_decoder_matches_product_distribution_fixture(golden, dtype, tol):
    fx = golden("product_distribution.json")
    addr = torch.tensor(fx["addr"], dtype=torch.float64).view(fx["shape"]).to(dtype)
    B, H = addr.shape[:2]
    pos = torch.tensor(fx["positions"])
    for case in fx["cases"]:
        idx, val = oracle.dense_topk_addr(addr, fx["embed_num"], pos, case["top_k"], case["re_norm"], dtype=dtype)
        got = _dense_map(idx, val, fx["A"], H)
        assert oracle.rel_err(got, torch.tensor(case["dense"], dtype=torch.float64).view(got.shape)) <= tol, case["top_k"]


def test_decoder_matches_extreme_logit_fixture(golden):
    fx = golden("extreme_logits.json")
    addr = torch.tensor(fx["addr"], dtype=torch.float64).view(fx["shape"])
    pos = torch.arange(addr.shape[-1]).view(1, -1)
    for case in fx["cases"]:
        idx, val = oracle.dense_topk_addr(addr, 0, pos, case["top_k"], case["re_norm"], dtype=torch.float64)
        got = _dense_map(idx, val, fx["A"], 1)[0, 0]
        torch.testing.assert_close(got, torch.tensor(case["dense"], dtype=torch.float64), atol=1e-12, rtol=1e-10)


@pytest.mark.parametrize("re_norm", [0.0, 0.5, 1.0])
@pytest.mark.parametrize("neg", [False, True])
def test_decoder_inactive_fixture(golden, re_norm, neg):
    fx = golden("inactive.json")
    addr = torch.tensor(fx["addr"]).view(fx["shape"])
    _, val = oracle.dense_topk_addr(addr, 1, torch.arange(3).expand(2, 3), 4, re_norm, neg)
    assert bool((val[..., :2] == 0).all()) and bool(torch.isfinite(val).all())
    assert bool((val[..., 2] != 0).any())


def _brute_force(addr, K, r):
    """Pure-Python brute force over all digit tuples for one address (U, P)."""
    U, P = len(addr), len(addr[0])
    logp = []
    for u in range(U):
        m = max(addr[u])
        z = math.log(sum(math.exp(x - m) for x in addr[u]))
        logp.append([x - m - z for x in addr[u]])
    scores = {}
    for digits in itertools.product(range(P), repeat=U):
        c = sum(d * P ** u for u, d in enumerate(digits))
        scores[c] = sum(logp[u][d] for u, d in enumerate(digits))
    top = sorted(scores, key=lambda c: (-scores[c], c))[:K]
    lse = math.log(sum(math.exp(scores[c]) for c in top))
    return {c: math.exp(scores[c] - r * lse) for c in top}


@pytest.mark.parametrize("U,P,K,r", [(3, 3, 5, 0.0), (2, 5, 7, 0.5), (4, 2, 3, 1.0), (1, 6, 2, 0.25)])
def test_decoder_matches_python_brute_force(U, P, K, r):
    g = torch.Generator().manual_seed(U * 10 + P)
    addr = torch.randn(1, 2, U, P, 3, generator=g, dtype=torch.float64)
    idx, val = oracle.dense_topk_addr(addr, 0, torch.zeros(1, 3, dtype=torch.long), K, r, dtype=torch.float64)
    A = P ** U
    for h in range(2):
        for t in range(3):
            want = _brute_force(addr[0, h, :, :, t].tolist(), K, r)
            got = {int(i) - h * A: float(v) for i, v in zip(idx[0, h, :, t], val[0, h, :, t])}
            assert set(got) == set(want)
            for c in want:
                assert math.isclose(got[c], want[c], rel_tol=1e-12)


def test_digit_significance_and_cape_direction():
    """Digit 0 is least significant; CAPE maps content c at position p to slot (c - p) mod A."""
    P, U = 4, 2
    A = P ** U
    addr = torch.full((1, 2, U, P, 1), -20.0)
    addr[0, :, 0, 1, 0] = 20.0  # digit 0 -> 1
    addr[0, :, 1, 2, 0] = 20.0  # digit 1 -> 2
    content = 1 + P * 2
    idx, _ = oracle.dense_topk_addr(addr, 1, torch.tensor([[7]]), 1, 0.0)
    assert int(idx[0, 0, 0, 0]) == (content - 7) % A          # head 0 shifted
    assert int(idx[0, 1, 0, 0]) == A + content                 # head 1 unshifted, batch-encoded base h*A


def test_index_checker_rejects_a_planted_mistake():
    case = make_case(1, 2, 2, 8, 16, 4, seed=21)
    idx, _ = oracle.dense_topk_addr(case.w_addr, 1, case.position_ids, 4)
    oracle.check_topk_indices(idx, case.w_addr, 1, case.position_ids, 4)
    scores, order = oracle.topk_f64(case.w_addr, 64)
    bad = idx.clone()
    # replace the best slot of one address by its 40th-ranked slot (far from a tie)
    shift = int(case.position_ids[0, 3]) % 64
    bad[0, 1, 0, 3] = 64 + (int(order[0, 1, 3, 40]) - 0) % 64  # head 1 has no CAPE shift
    del shift
    with pytest.raises(AssertionError):
        oracle.check_topk_indices(bad, case.w_addr, 1, case.position_ids, 4)


@pytest.mark.parametrize("t_chunk", [1, 5, 256])
def test_index_checker_rejects_mistakes_in_any_time_chunk(t_chunk):
    """The checker walks tokens in chunks: a wrong slot, a duplicated slot
    and an index outside its head's range are caught whichever chunk holds
    them, on CAPE and plain heads."""
    case = make_case(2, 2, 2, 8, 17, 4, seed=22)
    pos = case.position_ids * 3 + 5  # CAPE shifts beyond A
    idx, _ = oracle.dense_topk_addr(case.w_addr, 1, pos, 4)
    st = oracle.check_topk_indices(idx, case.w_addr, 1, pos, 4, t_chunk=t_chunk)
    assert st["addresses"] == 2 * 2 * 17
    _, order = oracle.topk_f64(case.w_addr, 64)
    for b, h, t in ((0, 0, 0), (1, 1, 16), (1, 0, 9)):
        base = (b * 2 + h) * 64
        shift = int(pos[b, t]) if h < 1 else 0
        wrong = idx.clone()
        wrong[b, h, 2, t] = base + (int(order[b, h, t, 50]) - shift) % 64  # the 51st-ranked slot
        dup = idx.clone()
        dup[b, h, 3, t] = dup[b, h, 0, t]
        out = idx.clone()
        out[b, h, 1, t] = base + 64 if (b, h) != (1, 1) else base - 1
        for bad in (wrong, dup, out):
            with pytest.raises(AssertionError):
                oracle.check_topk_indices(bad, case.w_addr, 1, pos, 4, t_chunk=t_chunk)


def test_index_checker_exempts_exact_ties():
    addr = torch.zeros(1, 1, 2, 4, 2)  # all 16 slots tie
    idx = torch.tensor([[[[15, 3], [2, 7], [9, 1], [4, 0]]]], dtype=torch.int32)
    st = oracle.check_topk_indices(idx, addr, 0, torch.zeros(1, 2, dtype=torch.long), 4)
    assert st["exempt_slots"] > 0


# ---------------------------------------------------------------------------
# gated sparse update closed forms

def _single_slot_events(w, r=None):
    """Events writing (and reading) slot 0 of a (1, 1, A) head at every token."""
    T = len(w)
    wi = torch.zeros(1, 1, 1, T, dtype=torch.int32)
    wv = torch.tensor(w, dtype=torch.float64).view(1, 1, 1, T)
    rv = torch.ones(1, 1, 1, T, dtype=torch.float64) if r is None else torch.tensor(r, dtype=torch.float64).view(1, 1, 1, T)
    return wi, wv, wi.clone(), rv


def _run_both(events, x, gamma, slot0, mass0, mass_aware=False, A=4):
    """The sparse fp64 loop and the dense fp32 loop on the same decoded events."""
    wi, wv, ri, rv = events
    sp = oracle.sparse_gsu_f64(wi, wv, ri, rv, x, gamma, slot0, mass0, None, mass_aware, 1e-12)
    T = x.shape[2]
    dummy = torch.zeros(1, 1, 1, A, T)
    de = oracle.dense_ram_attn(dummy, dummy, x.float(), gamma.float(), slot0.float(), mass0.float(), None, 0, None,
                               (wi.shape[2], ri.shape[2]), (0.0, 0.0), mass_aware, 1e-12,
                               decoded=(wi, wv.float(), ri, rv.float()))
    return sp, de


def test_gsu_pure_accumulation_is_a_weighted_mean():
    """gamma -> -inf gives alpha = 1: the slot is the mass-weighted mean of its writes."""
    g = torch.Generator().manual_seed(1)
    T, C = 12, 5
    w = (torch.rand(T, generator=g, dtype=torch.float64) * 0.9 + 0.05).tolist()
    x = torch.randn(1, 1, T, C, generator=g, dtype=torch.float64)
    gamma = torch.full((1, 1, T), -80.0, dtype=torch.float64)
    s0 = torch.randn(1, 1, 4, C, generator=g, dtype=torch.float64)
    m0 = torch.full((1, 1, 4), 0.3, dtype=torch.float64)
    (y, s, m), (yd, sd, md) = _run_both(_single_slot_events(w), x, gamma, s0, m0)
    wt = torch.tensor(w, dtype=torch.float64)
    cum_m = 0.3 + torch.cumsum(wt, 0)
    cum_x = 0.3 * s0[0, 0, 0] + torch.cumsum(wt[:, None] * x[0, 0], 0)
    expect_y = cum_x / cum_m[:, None]
    assert np.allclose(y[0, 0], expect_y.numpy(), rtol=1e-10, atol=1e-12)
    assert math.isclose(m[0, 0, 0], float(cum_m[-1]), rel_tol=1e-12)
    assert oracle.rel_err(yd[0, 0], expect_y) <= 1e-5 and oracle.rel_err(sd[0, 0, 0], expect_y[-1]) <= 1e-5


def test_gsu_full_forgetting_keeps_the_last_write():
    """gamma -> +inf gives alpha = 0: mass = w and the slot equals the last written value."""
    g = torch.Generator().manual_seed(2)
    T, C = 6, 3
    w = [0.3, 0.5, 0.2, 0.9, 0.4, 0.7]
    x = torch.randn(1, 1, T, C, generator=g, dtype=torch.float64)
    gamma = torch.full((1, 1, T), 80.0, dtype=torch.float64)
    s0 = torch.randn(1, 1, 4, C, generator=g, dtype=torch.float64)
    m0 = torch.ones(1, 1, 4, dtype=torch.float64)
    (y, s, m), (yd, sd, md) = _run_both(_single_slot_events(w), x, gamma, s0, m0)
    assert np.allclose(y[0, 0], x[0, 0].numpy(), rtol=1e-10)
    assert math.isclose(m[0, 0, 0], w[-1], rel_tol=1e-12)
    assert oracle.rel_err(yd[0, 0], x[0, 0]) <= 1e-5


def test_gsu_constant_weight_mass_is_geometric():
    """Constant w and gamma: m_n = a^n m_0 + w (1 - a^n) / (1 - a), a = (1 - w) / (1 - w + e^gamma w)."""
    T, C, w, gam, m_0 = 20, 2, 0.25, 0.4, 0.7
    x = torch.zeros(1, 1, T, C, dtype=torch.float64)
    gamma = torch.full((1, 1, T), gam, dtype=torch.float64)
    a = (1 - w) / (1 - w + math.exp(gam) * w)
    s0 = torch.zeros(1, 1, 4, C, dtype=torch.float64)
    m0 = torch.full((1, 1, 4), m_0, dtype=torch.float64)
    (y, s, m), (yd, sd, md) = _run_both(_single_slot_events([w] * T), x, gamma, s0, m0)
    expect = a ** T * m_0 + w * (1 - a ** T) / (1 - a)
    assert math.isclose(m[0, 0, 0], expect, rel_tol=1e-12)
    assert math.isclose(float(md[0, 0, 0]), expect, rel_tol=1e-5)


def test_mass_aware_read_closed_form():
    """Two read slots: y = (r1 + r2) (m1 r1 s1 + m2 r2 s2) / (m1 r1 + m2 r2 + eps); no writes (w = 0)."""
    C = 3
    s0 = torch.tensor([[[[1.0, 2.0, 3.0], [-1.0, 0.5, 4.0], [0.0, 0.0, 0.0], [0.0, 0.0, 0.0]]]], dtype=torch.float64)
    m0 = torch.tensor([[[0.2, 1.5, 1.0, 1.0]]], dtype=torch.float64)
    wi = torch.zeros(1, 1, 1, 1, dtype=torch.int32)
    wv = torch.zeros(1, 1, 1, 1, dtype=torch.float64)
    ri = torch.tensor([0, 1], dtype=torch.int32).view(1, 1, 2, 1)
    rv = torch.tensor([0.6, 0.3], dtype=torch.float64).view(1, 1, 2, 1)
    x = torch.zeros(1, 1, 1, C, dtype=torch.float64)
    gamma = torch.zeros(1, 1, 1, dtype=torch.float64)
    (y, _, _), (yd, _, _) = _run_both((wi, wv, ri, rv), x, gamma, s0, m0, mass_aware=True)
    num = 0.6 * 0.2 * s0[0, 0, 0] + 0.3 * 1.5 * s0[0, 0, 1]
    expect = 0.9 * num / (0.6 * 0.2 + 0.3 * 1.5 + 1e-12)
    assert np.allclose(y[0, 0, 0], expect.numpy(), rtol=1e-12)
    assert oracle.rel_err(yd[0, 0, 0], expect) <= 1e-6


# ---------------------------------------------------------------------------
# the two algorithms agree; behavioural invariants

@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("mass_aware", [False, True])
@pytest.mark.parametrize("top_k,re_norm", [((4, 4), (0.0, 0.0)), ((4, 12), (0.25, 0.75)), ((8, 8), (1.0, 1.0))])
def test_dense_and_sparse_algorithms_agree(masked, mass_aware, top_k, re_norm):
    case = make_case(2, 3, 3, 3, 29, 6, seed=17, masked=masked)
    y, s, m = oracle.dense_ram_attn(case.w_addr, case.r_addr, case.values, case.gamma, case.init_slot,
                                    case.init_mass, case.mask, 2, case.position_ids, top_k, re_norm, mass_aware, 1e-12)
    wi, wv = oracle.dense_topk_addr(case.w_addr, 2, case.position_ids, top_k[0], re_norm[0])
    ri, rv = oracle.dense_topk_addr(case.r_addr, 2, case.position_ids, top_k[1], re_norm[1])
    ys, ss, ms = oracle.sparse_gsu_f64(wi, wv, ri, rv, case.values, case.gamma, case.init_slot, case.init_mass,
                                       case.mask, mass_aware, 1e-12)
    keep = torch.ones(29, dtype=torch.bool) if case.mask is None else case.mask[0]
    assert oracle.rel_err(y[:, :, keep], torch.as_tensor(ys)[:, :, keep]) <= 1e-5
    assert oracle.rel_err(s, ss) <= 1e-5 and oracle.rel_err(m, ms) <= 1e-5


@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("mass_aware", [False, True])
@pytest.mark.parametrize("gamma_scale", [0.5, 6.0])
def test_sparse_backward_matches_dense_autograd(masked, mass_aware, gamma_scale):
    """The state-reconstruction backward against fp64 torch autograd through
    the dense restatement on the same events. Some weights are zeroed: such
    events do not act and their gradient is 0 by contract (autograd's value
    there is masked out before comparing)."""
    case = make_case(2, 3, 2, 4, 31, 5, seed=23, masked=masked, gamma_scale=gamma_scale)
    Kw, Kr = 3, 4
    wi, wv = oracle.dense_topk_addr(case.w_addr, 1, case.position_ids, Kw, 0.5, dtype=torch.float64)
    ri, rv = oracle.dense_topk_addr(case.r_addr, 1, case.position_ids, Kr, 0.0, dtype=torch.float64)
    wv, rv = wv.clone(), rv.clone()
    wv[..., ::7] = 0.0
    rv[:, :, 1, ::5] = 0.0
    gen = torch.Generator().manual_seed(5)
    Dy = torch.randn(case.values.shape, generator=gen, dtype=torch.float64)
    Ds = torch.randn(case.init_slot.shape, generator=gen, dtype=torch.float64)
    Dm = torch.randn(case.init_mass.shape, generator=gen, dtype=torch.float64)
    got = oracle.sparse_gsu_backward_f64(wi, wv, ri, rv, case.values, case.gamma, case.init_slot, case.init_mass, Dy,
                                         Ds, Dm, case.mask, mass_aware, 1e-12)
    wl = wv.double().requires_grad_(True)
    rl = rv.double().requires_grad_(True)
    leaves = [t.double().requires_grad_(True) for t in (case.values, case.gamma, case.init_slot, case.init_mass)]
    y, s, m = oracle.dense_ram_attn(case.w_addr.double(), case.r_addr.double(), *leaves, case.mask, 0, None,
                                    (Kw, Kr), (0.0, 0.0), mass_aware, 1e-12, decoded=(wi, wl, ri, -rl))
    keep = torch.ones(2, 31, dtype=torch.float64) if case.mask is None else case.mask.double()
    ((y * Dy * keep[:, None, :, None]).sum() + (s * Ds).sum() + (m * Dm).sum()).backward()
    ref = [wl.grad.masked_fill(wv == 0, 0), rl.grad.masked_fill(rv == 0, 0)] + [t.grad for t in leaves]
    for name, a, b in zip(("w", "r", "x", "gamma", "slot", "mass"), got, ref):
        assert b.abs().max() > 0, f"{name}: the reference gradient is zero, so the comparison would be vacuous"
        assert oracle.rel_err(torch.as_tensor(a), b) <= 1e-9, name


def test_dense_oracle_is_chunk_invariant():
    case = make_case(1, 2, 2, 4, 40, 4, seed=3, masked=True)
    args = (case.w_addr, case.r_addr, case.values, case.gamma, case.init_slot, case.init_mass, case.mask, 1,
            case.position_ids, (4, 4), (0.5, 0.5), True, 1e-12)
    full = oracle.dense_ram_attn(*args, chunk=256)
    for chunk in (1, 7, 13):
        part = oracle.dense_ram_attn(*args, chunk=chunk)
        for a, b in zip(full, part):
            # torch's CPU kernels vectorise by shape, so only rounding may differ
            assert oracle.rel_err(b, a) <= 1e-6


def test_sparse_oracle_steps_match_one_call_and_masked_tokens_are_skipped():
    case = make_case(2, 2, 2, 4, 15, 5, seed=8, masked=True)
    wi, wv = oracle.dense_topk_addr(case.w_addr, 1, case.position_ids, 3)
    ri, rv = oracle.dense_topk_addr(case.r_addr, 1, case.position_ids, 5)
    y, s, m = oracle.sparse_gsu_f64(wi, wv, ri, rv, case.values, case.gamma, case.init_slot, case.init_mass, case.mask)
    st, mt = case.init_slot, case.init_mass
    ys = []
    for t in range(15):
        yt, st, mt = oracle.sparse_gsu_f64(wi[..., t:t + 1], wv[..., t:t + 1], ri[..., t:t + 1], rv[..., t:t + 1],
                                           case.values[:, :, t:t + 1], case.gamma[..., t:t + 1], st, mt,
                                           case.mask[:, t:t + 1])
        ys.append(yt)
    assert np.allclose(np.concatenate(ys, axis=2), y, rtol=0, atol=0)
    assert np.array_equal(st, s) and np.array_equal(mt, m)
    keep = case.mask[0].numpy()
    assert np.all(y[:, :, ~keep] == 0)
    # compacting the valid tokens (positions unchanged) gives the same state
    k = case.mask[0]
    yc, sc, mc = oracle.sparse_gsu_f64(wi[..., k], wv[..., k], ri[..., k], rv[..., k], case.values[:, :, k],
                                       case.gamma[..., k], case.init_slot, case.init_mass)
    assert np.allclose(yc, y[:, :, keep], rtol=0, atol=0) and np.array_equal(sc, s)


def test_rel_err():
    assert oracle.rel_err(torch.tensor([1.0, 2.0]), torch.tensor([1.0, 4.0])) == 0.5
    assert oracle.rel_err(torch.zeros(3), torch.zeros(3)) == 0.0

"""The exact paths ``bench.py`` times, at the benchmark configurations,
against the CPU oracle.

* Configs 2 and 4 (plain and tie-heavy): the record decoder
  (``ramnet_topk_addr_records``) followed by ``ramnet_segment_scan``, called
  through the C ABI exactly as the benchmark calls them, on the benchmark's
  own inputs (``bench.make_prefill_inputs``). Its per-event records must
  equal, bit for bit, the records ``pack_records_kernel`` builds from
  ``ramnet_topk_addr_forward``'s (idx, val) -- slot, weight and forget
  coefficient -- the packer's per-token overlap flags (bit d - 1: a written
  slot shared with token t - d, d = 1..3) must equal the exact ones computed
  here from the slots, and the record decoder's must be set wherever those
  are (it may also be set where they are not: a wave's first lanes assume
  overlap). The indices of every token, and y, slot and mass of every head,
  match the fp64 ranking and the fp64 event loop.
* Config 3: 16 consecutive decode steps at B=64, H=16 on the 64x16x1024x128
  fp32 state, captured in one HIP graph as the benchmark captures them and
  replayed; every step's indices against the fp64 ranking, and y of every
  step plus the whole state of several (b, h) heads against the stepwise
  fp64 event loop.
* A scan only reads its records: two scans from one set of records give the
  same bits, in the mass-wave form and in the precomputed-gain form.

Bars: indices bit-exact except fp64 ties within 1e-6; fp32 state
rel <= 1e-5; bf16 outputs rel <= 2e-2 (max|a-b| / max|b|).
"""
from __future__ import annotations

import pytest
import torch

import oracle
from ram_cases import make_case

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
LOW_TOL = 2e-2
DEV = "cuda"


def _nat():
    import ramnet_ops  # noqa: F401  (registers torch.ops.ramnet_ops.*)
    from ramnet_ops import _native
    _native.lib()
    return _native


def _records(ws: torch.Tensor, B: int, H: int, T: int, Kw: int, Kr: int):
    """Views of a scan workspace: write records (B*H, Kw, T_pad, 4) and read
    records (B*H, Kr, T_pad, 2), as int32 words."""
    tp = (T + 31) // 32 * 32
    wb = B * H * Kw * tp * 16
    rb = B * H * Kr * tp * 8
    w = ws[:wb].view(torch.int32).view(B * H, Kw, tp, 4)
    r = ws[wb:wb + rb].view(torch.int32).view(B * H, Kr, tp, 2)
    return w, r


# the prefill configurations bench.py times, by test id
PREFILL = {"config2": "C2", "config4": "C4", "config4_tie_heavy": "C4_TIES"}


@pytest.fixture(scope="module", params=list(PREFILL))
def timed_prefill(request):
    """One run of a benchmarked prefill path at its full size, two ways:
    (a) ``ramnet_topk_addr_records`` then ``ramnet_segment_scan``, called as
    ``bench.bench_prefill`` calls them on ``bench.make_prefill_inputs``'s
    inputs; (b) ``topk_addr_forward``'s (idx, val) packed into records by
    ``ramnet_topk_segment_forward``. Everything stays on the GPU."""
    import bench  # the benchmark's configurations and input builder
    nat = _nat()
    ops = torch.ops.ramnet_ops
    c = getattr(bench, PREFILL[request.param])
    B, H, T, C, U, P, K, E = (c[k] for k in ("B", "H", "T", "C", "U", "P", "K", "embed"))
    A = P ** U
    print(f"{request.param}: benched prefill path at full size B={B} H={H} T={T} A={A} K={K}"
          f"{' quantised logits' if c['quant'] else ''}", flush=True)
    host, d = bench.make_prefill_inputs(DEV, c)
    slot0 = torch.zeros(B, H, A, C, device=DEV)
    mass0 = torch.full((B, H, A), 1.0 / A, device=DEV)
    n = nat.scan_workspace_bytes(B, H, T, K, K)
    code = nat.DTYPE_CODES[torch.bfloat16]
    stream = torch.cuda.current_stream().cuda_stream
    # (a) the benchmark's two calls
    ws_a = torch.empty(n, dtype=torch.uint8, device=DEV)
    out_a = (torch.empty_like(d["x"]), torch.empty_like(slot0), torch.empty_like(mass0))
    nat.call("ramnet_topk_addr_records", d["w"].data_ptr(), d["r"].data_ptr(), d["gamma"].data_ptr(), code, None,
             E, d["pos"].data_ptr(), B, H, U, P, T, A, K, K, 0.0, 0.0, ws_a.data_ptr(), n, stream)
    nat.call("ramnet_segment_scan", d["x"].data_ptr(), code, slot0.data_ptr(), mass0.data_ptr(),
             out_a[1].data_ptr(), out_a[2].data_ptr(), out_a[0].data_ptr(), B, H, T, A, C, K, K, 0, 1e-12,
             ws_a.data_ptr(), n, stream)
    # (b) decoder outputs, packed into records by the segment op
    idx, val = ops.topk_addr_forward(d["w"], d["r"], E, A, d["pos"], K, K, 0.0, 0.0)
    ws_b = torch.empty(n, dtype=torch.uint8, device=DEV)
    out_b = (torch.empty_like(d["x"]), torch.empty_like(slot0), torch.empty_like(mass0))
    nat.call("ramnet_topk_segment_forward", idx.data_ptr(), val.data_ptr(), d["x"].data_ptr(), d["gamma"].data_ptr(),
             code, None, slot0.data_ptr(), mass0.data_ptr(), out_b[1].data_ptr(), out_b[2].data_ptr(),
             out_b[0].data_ptr(), B, H, T, A, C, K, K, 0, 1e-12, ws_b.data_ptr(), n, stream)
    torch.cuda.synchronize()
    yield dict(name=request.param, dims=(B, H, T, C, U, P, K, E, A), host=host, ws_a=ws_a, ws_b=ws_b, out_a=out_a,
               out_b=out_b, idx=idx, val=val)


def test_timed_prefill_records_match_packed_records(timed_prefill):
    """Record-mode decoder records == records packed from (idx, val): slot,
    weight and forget coefficient bit for bit; the packer's overlap flags
    (bit d - 1: a written slot shared with token t - d, d = 1..3, exact for
    top-K <= 16) equal the flags computed here from the slots; the record
    decoder's flags are a superset (a wave's first lanes assume overlap);
    and both scans give the same bits (the flags only select a reload)."""
    run = timed_prefill
    B, H, T, C, U, P, K, E, A = run["dims"]
    wa, ra = _records(run["ws_a"], B, H, T, K, K)
    wb, rb = _records(run["ws_b"], B, H, T, K, K)
    assert torch.equal(wa[..., :3], wb[..., :3]), "write records (slot, w, alpha) differ from the packed records"
    assert torch.equal(ra, rb), "read records (slot, r) differ from the packed records"
    fa, fb = wa[:, 0, :T, 3], wb[:, 0, :T, 3]
    slots = wb[:, :, :T, 0]  # (B*H, K, T), -2 for no-op writes
    exact = torch.zeros_like(fb)
    for dd in (1, 2, 3):
        cur, prev = slots[:, :, None, dd:], slots[:, None, :, :-dd]
        hit = ((cur == prev) & (cur >= 0)).flatten(1, 2).any(dim=1)
        exact[:, dd:] |= hit.to(exact.dtype) << (dd - 1)
    assert torch.equal(fb, exact), "packed-record overlap flags differ from the exact ones (top-K <= 16)"
    assert bool(((fa & exact) == exact).all()), "record-mode overlap flag missing where the write sets overlap"
    print(f"{run['name']}: overlap flags (t-1, t-2, t-3): record mode "
          f"{[int(((fa >> k) & 1).sum()) for k in range(3)]}, exact {[int(((exact >> k) & 1).sum()) for k in range(3)]}"
          f" of {B * H * T} tokens", flush=True)
    for name, a, b in zip(("y", "slot", "mass"), run["out_a"], run["out_b"]):
        assert torch.equal(a, b), f"{name}: the benched path differs from the packed-record path"


def test_timed_prefill_indices_every_token(timed_prefill):
    """Write and read indices of every address against the fp64 ranking of
    the same logits (ties within 1e-6 exempt), in chunks of 256 tokens."""
    run = timed_prefill
    B, H, T, C, U, P, K, E, A = run["dims"]
    host = run["host"]
    idx_c = run["idx"].cpu()
    pos = host["pos"].long()
    for lg, rows, what in ((host["w"], slice(0, K), "write"), (host["r"], slice(K, 2 * K), "read")):
        st = oracle.check_topk_indices(idx_c[:, :, rows], lg, E, pos, K, t_chunk=256)
        print(f"{run['name']} {what}: {st['addresses']} addresses, {st['exempt_slots']} tie-exempt slots",
              flush=True)


def _worst_head_rel(a, b) -> float:
    """max over (b, h) of max|a - b| / max|b| within the head."""
    a = torch.as_tensor(a).double().flatten(2)
    b = torch.as_tensor(b).double().flatten(2)
    num = (a - b).abs().amax(-1)
    den = b.abs().amax(-1).clamp_min(1e-300)
    return float((num / den).max())


def test_timed_prefill_outputs_every_head(timed_prefill):
    """y, slot and mass of every (b, h) head against the fp64 event loop on
    the decoder's events (fp32 state rel <= 1e-5, bf16 y rel <= 2e-2, per
    head)."""
    run = timed_prefill
    B, H, T, C, U, P, K, E, A = run["dims"]
    host = run["host"]
    wi, wv, ri, rv = oracle.split_events(run["idx"].cpu(), run["val"].cpu(), K)
    ry, rslot, rmass = oracle.sparse_gsu_f64(wi, wv, ri, rv, host["x"].double(), host["gamma"].double(),
                                             torch.zeros(B, H, A, C), torch.full((B, H, A), 1.0 / A), None, False,
                                             1e-12)
    y, slot, mass = (t.cpu() for t in run["out_a"])
    errs = {"slot": _worst_head_rel(slot, rslot), "mass": _worst_head_rel(mass.unsqueeze(-1), rmass[..., None]),
            "y": _worst_head_rel(y, ry)}
    print(f"{run['name']}: worst-head rel err over {B * H} heads {errs}", flush=True)
    assert errs["slot"] <= FP32_TOL and errs["mass"] <= FP32_TOL, errs
    assert errs["y"] <= LOW_TOL, errs


def test_config3_graph_captured_steps_match_oracle():
    """Config 3 decode as the benchmark runs it (bench.py bench_decode): the
    steps captured in one HIP graph, replayed on the persistent state."""
    _nat()
    ops = torch.ops.ramnet_ops
    B, H, C, U, P, K, S = 64, 16, 128, 2, 32, 8, 16
    A = P ** U
    E = H // 2
    print(f"config 3: {S} graph-captured decode steps at B={B}, H={H}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(3)
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
    ys = []

    def run_all():
        ys.clear()
        for s in range(S):
            ys.append(ops.topk_autoregressive_(w_all[s], r_all[s], x_all[s], g_all[s], slot, mass, no_mask, E,
                                               pos_all[s], K, K, 0.0, 0.0, False, 1e-12))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run_all()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_all()
    torch.cuda.synchronize()

    heads = ((0, 0), (17, 5), (33, 8), (63, 15), (40, 12))
    sel = lambda t: torch.stack([t[b, h] for b, h in heads]).unsqueeze(1).cpu()  # (n, 1, ...)
    slot_before, mass_before = sel(slot), sel(mass)
    graph.replay()
    torch.cuda.synchronize()
    y_steps = torch.stack([y.cpu() for y in ys], dim=2)  # (B, H, S, C)
    slot_after, mass_after = sel(slot), sel(mass)

    # every step's indices (all B x H addresses) against the fp64 ranking;
    # the same decoder gives the events of the heads checked below
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
    y_sel = sel(y_steps)  # (n, 1, S, C)
    for s in range(S):
        err = oracle.rel_err(y_sel[:, :, s], ry[:, :, s])
        assert err <= LOW_TOL, f"y of step {s}: rel err {err:.3e}"
    assert oracle.rel_err(slot_after, rslot) <= FP32_TOL, "slot state after the captured steps"
    assert oracle.rel_err(mass_after, rmass) <= FP32_TOL, "mass state after the captured steps"
    touched = (slot_after != slot_before).any(-1)
    print(f"rows changed per checked head: {touched.sum(-1).flatten().tolist()}", flush=True)


@pytest.mark.parametrize("layout,pre", [("1,16,1,1", False), ("1,16,1,2,1", True)],
                         ids=["mass_wave", "precomputed_gains"])
def test_scan_reads_records_only(layout, pre, monkeypatch):
    """``ramnet_segment_scan`` run twice on one set of records from
    ``ramnet_topk_addr_records`` gives identical outputs, and both match the
    fp64 event loop: the precomputed-gain form writes its gains to its own
    part of the workspace, never into the decoder records."""
    nat = _nat()
    monkeypatch.setenv("RAMNET_SCAN_LAYOUT", layout)
    B, H, U, P, T, C, K, E = 2, 2, 3, 16, 700, 64, 8, 1
    A = P ** U
    plan = nat.segment_plan(B, H, A, C, K, K, torch.bfloat16)
    assert plan is not None and plan[2] == pre, plan
    print(f"scan twice from one record set, layout {layout} {plan}", flush=True)
    case = make_case(B, H, U, P, T, C, dtype=torch.bfloat16, seed=71, masked=True)
    d = case.to(DEV)
    pos = d.position_ids.to(torch.int32).contiguous()
    mask = d.mask.to(torch.uint8).contiguous()
    n = nat.scan_workspace_bytes(B, H, T, K, K)
    ws = torch.empty(n, dtype=torch.uint8, device=DEV)
    code = nat.DTYPE_CODES[torch.bfloat16]
    stream = torch.cuda.current_stream().cuda_stream
    nat.call("ramnet_topk_addr_records", d.w_addr.data_ptr(), d.r_addr.data_ptr(), d.gamma.data_ptr(), code,
             mask.data_ptr(), E, pos.data_ptr(), B, H, U, P, T, A, K, K, 0.0, 0.0, ws.data_ptr(), n, stream)
    w0, r0 = (t.clone() for t in _records(ws, B, H, T, K, K))
    outs = []
    for _ in range(2):
        slot, mass, y = torch.empty_like(d.init_slot), torch.empty_like(d.init_mass), torch.empty_like(d.values)
        nat.call("ramnet_segment_scan", d.values.data_ptr(), code, d.init_slot.data_ptr(), d.init_mass.data_ptr(),
                 slot.data_ptr(), mass.data_ptr(), y.data_ptr(), B, H, T, A, C, K, K, 0, 1e-12, ws.data_ptr(), n,
                 stream)
        outs.append((y, slot, mass))
    torch.cuda.synchronize()
    w1, r1 = _records(ws, B, H, T, K, K)
    assert torch.equal(w0, w1) and torch.equal(r0, r1), "the scan modified the decoder records"
    for a, b in zip(*outs):
        assert torch.equal(a, b), "second scan of the same records differs"
    # the events those records hold, from the decoder op on the same inputs
    idx, val = torch.ops.ramnet_ops.topk_addr_forward(d.w_addr, d.r_addr, E, A, d.position_ids, K, K, 0.0, 0.0)
    wi, wv, ri, rv = oracle.split_events(idx.cpu(), val.cpu(), K)
    ry, rslot, rmass = oracle.sparse_gsu_f64(wi, wv, ri, rv, case.values.double(), case.gamma.double(),
                                             case.init_slot, case.init_mass, case.mask)
    y, slot, mass = (t.cpu() for t in outs[0])
    keep = case.mask[0]
    assert bool((y[:, :, ~keep] == 0).all())
    assert oracle.rel_err(slot, rslot) <= FP32_TOL
    assert oracle.rel_err(mass, rmass) <= FP32_TOL
    assert oracle.rel_err(y[:, :, keep], torch.as_tensor(ry)[:, :, keep]) <= LOW_TOL

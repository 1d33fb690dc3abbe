"""Benchmark of the RAM-Net operator hot path on one MI355X.

Headline (``value``): segment-parallel prefill tokens/s at config 2
(B=8, H=16, T=4096, d_v=128, U=2, P=32 -> A=1024 slots, K=8, bf16
activations, fp32 slot state, CAPE on half the heads). One step = the address
decoder for write and read logits plus the segment scan (GSU + top-K read)
over the whole batch, inputs resident in HBM, functional state
(zeros in, new state out). The decode figure (config 3: B=64, 512 fused
single-token steps on a persistent 64x16x1024x128 fp32 state, captured in a
HIP graph, one launch per step) is reported beside it under ``decode``, with
the labelled multi-step variant (the same 512 steps in one persistent launch
of ``topk_autoregressive_steps_``) under ``decode.multi_step``. Timings give
the median, min and max over repetitions. Config 1 (fp32, one fused forward
call) is reported under ``config1``.

``roofline`` is for the dominant stage (the segment stage: mass pre-pass and
segment scan, one C-ABI call), timed with HIP events on the stream it runs
on: ``achieved`` / ``frac`` are its counter-measured HBM bytes per call
(rocprofv3, ``--traffic-summary``) over that time against the HBM peak;
``bound`` names what binds it (LDS: the slot state stays on chip), with the
slot-row bytes it moves through LDS priced against an LDS read peak measured
in the same run, and the event ("active state") model's figure beside them. ``cpu_baseline`` times the CPU
restatement of the reference's dense PyTorch algorithm on a bounded sample of
the same config-2 inputs (rank 0, N=1 only); ``cpu_baselines`` does the same
for config 1 (in full), config 3 (32 consecutive decode steps) and config 4
(512 tokens), each with the host CPU's model string.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--decode-steps S]
       [--no-cpu-baseline] [--no-stress] [--no-lm] [--lm-tokens N]
       [--only prefill|decode|stress|lm|train] [--no-train] [--copy-probe MIB]
       [--traffic-summary DIR]

Config 4 (B=4, H=8, T=8192, U=3, P=16 -> A=4096, K=16) and its tie-heavy
variant (decoder logits quantised to multiples of 0.25) are timed the same
way and reported under ``stress``. Config 5 (the caller harness: a 24-block
RAM-Net LM, prompt 16 x 2048, greedy in-place decode) is reported under
``lm``. A config-2 training step of the operator (differentiable forward,
then the segment and decoder backward) is reported under ``train``.

``--copy-probe MIB`` first runs one plain device-to-device copy of MIB MiB
(torch ``copy_``, fp32): under ``rocprofv3 --pmc FETCH_SIZE`` / ``WRITE_SIZE``
it is the calibration kernel of known traffic for the byte counters.
"""
from __future__ import annotations

import argparse
import csv
import hashlib
import json
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(REPO, "ram-net_amd"), REPO, os.path.join(REPO, "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
# Counter-measured HBM bytes per call of the prefill stages at configs 2 and
# 4: rocprofv3 FETCH_SIZE / WRITE_SIZE passes over this script, calibrated on
# a copy of known size and written by `bench.py --traffic-summary DIR`. The
# file records a digest of the kernel sources it was measured with; a line
# built from other sources reports it as stale.
TRAFFIC_FILE = os.path.join(REPO, "profiles", "segment_stage_traffic.json")
TRAFFIC_SOURCES = ("segment_scan.hpp", "segment_scan_pair.hpp", "segment_forward.hip", "segment_scan_bf16.hip",
                   "ramnet_kernels.hpp", "ramnet_device.hpp", "topk_addr.hip", "lane_search.hpp", "capi.hip")
# the scan kernels of the segment stage (one-token, paired, slot-range forms)
SCAN_KERNELS = ("segment_scan_kernel", "segment_scan_pair_kernel", "segment_scan_range_kernel")
PROBE_LIB = os.path.join(REPO, "ram-net_amd", "ramnet_ops", "_lib", "libramnet_lds_probe.so")
METRIC = "prefill tokens/s (T=4096) + decode tokens/s (B=64); % HBM roofline"

# config 2 (prefill), config 3 (decode), config 4 (stress prefill; tie-heavy
# variant: decoder logits quantised to multiples of 0.25)
C2 = dict(B=8, H=16, T=4096, C=128, U=2, P=32, K=8, d_k=128, seed=2, embed=8, gamma_shift=-1.0, quant=None)
C3 = dict(B=64, H=16, C=128, U=2, P=32, K=8, steps=512, seed=3)
C4 = dict(B=4, H=8, T=8192, C=128, U=3, P=16, K=16, d_k=128, seed=4, embed=4, gamma_shift=0.0, quant=None)
C4_TIES = dict(C4, quant=0.25)
# config 5 (caller harness): a 24-block RAM-Net LM, prompt 16 x 2048, then
# greedy single-token steps with in-place per-layer state
C5 = dict(layers=24, d_model=1024, heads=8, C=128, U=2, P=32, K=8, vocab=32000, embed=4, mlp=2816, B=16, T=2048,
          new=256, seed=5)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def source_digest() -> str:
    """Digest of the kernel sources the prefill traffic depends on."""
    h = hashlib.sha256()
    for name in TRAFFIC_SOURCES:
        with open(os.path.join(REPO, "ram-net_amd", "csrc", name), "rb") as f:
            h.update(name.encode() + b"\0" + f.read())
    return h.hexdigest()[:16]


def load_traffic() -> dict | None:
    """The counter-measured traffic file, with ``current`` telling whether it
    was measured on the kernel sources of this tree."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as f:
        tr = json.load(f)
    tr["current"] = tr.get("source_digest") == source_digest()
    return tr


def lds_read_peak(dev, reps=5) -> dict | None:
    """LDS read bandwidth of the whole GPU, measured live: a conflict-free
    ds_read_b128 stream (csrc/lds_probe.hip), five workgroups of 256 threads
    per CU, timed with HIP events on the stream it runs on; best of ``reps``."""
    import ctypes
    if not os.path.exists(PROBE_LIB):
        return None
    lib = ctypes.CDLL(PROBE_LIB)
    lib.ramnet_lds_probe.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.ramnet_lds_probe.restype = ctypes.c_int
    lib.ramnet_lds_probe_bytes.argtypes = [ctypes.c_int, ctypes.c_int]
    lib.ramnet_lds_probe_bytes.restype = ctypes.c_int64
    n_cu = torch.cuda.get_device_properties(dev).multi_processor_count
    blocks, iters = 5 * n_cu, 4096
    sink = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    best = None
    for _ in range(reps + 1):  # the first launch warms up
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        rc = lib.ramnet_lds_probe(blocks, iters, ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(stream))
        e1.record()
        torch.cuda.synchronize()
        if rc != 0:
            return None
        ms = e0.elapsed_time(e1)
        best = ms if best is None else min(best, ms)
    nbytes = lib.ramnet_lds_probe_bytes(blocks, iters)
    return {"gbs": nbytes / (best / 1e3) / 1e9, "cus": n_cu, "bytes": nbytes, "ms": best,
            "kernel": "lds_read_probe_kernel (ds_read_b128, no bank conflicts)"}


def traffic_summary(out_dir: str) -> int:
    """Write TRAFFIC_FILE from rocprofv3 runs in ``out_dir``: for w in
    (prefill, stress), ``<w>_trace`` (--kernel-trace --stats) and
    ``<w>_FETCH_SIZE`` / ``<w>_WRITE_SIZE`` (--pmc) of ``bench.py --only <w>
    --copy-probe 1024``. FETCH_SIZE and WRITE_SIZE (KiB per dispatch,
    medians) are scaled by what they read for the 1 GiB copy."""
    import statistics
    stage_names = SCAN_KERNELS + ("segment_mass_kernel", "mass_chunk_map_kernel", "mass_chunk_scan_kernel")

    def counters(path):
        vals = {}
        with open(path) as f:
            for r in csv.DictReader(f):
                vals.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
        return {k: statistics.median(v) for k, v in vals.items()}

    res = {"source_digest": source_digest(), "unit": "bytes per call", "configs": {}}
    for w, name in (("prefill", "config2"), ("stress", "config4")):
        fe = counters(os.path.join(out_dir, f"{w}_FETCH_SIZE", "run_counter_collection.csv"))
        wr = counters(os.path.join(out_dir, f"{w}_WRITE_SIZE", "run_counter_collection.csv"))
        fs = 1048576.0 / next(v for k, v in fe.items() if "copyBuffer" in k)
        ws = 1048576.0 / next(v for k, v in wr.items() if "copyBuffer" in k)
        with open(os.path.join(out_dir, f"{w}_trace", "run_kernel_stats.csv")) as f:
            trace = {r["Name"]: float(r["AverageNs"]) / 1e3 for r in csv.DictReader(f)}
        part = {"scan": 0.0, "prepass": 0.0, "decoder": 0.0}
        times = {"scan": 0.0, "prepass": 0.0, "decoder": 0.0}
        for k, v in fe.items():
            which = ("scan" if any(n in k for n in SCAN_KERNELS) else "prepass" if any(n in k for n in stage_names)
                     else "decoder" if "topk_addr" in k else None)
            if which is None:
                continue
            part[which] += (v * fs + wr.get(k, 0.0) * ws) * 1024
            times[which] += next((t for n, t in trace.items() if n == k), 0.0)
        res["configs"][name] = {
            "scan_bytes": part["scan"], "prepass_bytes": part["prepass"], "decoder_bytes": part["decoder"],
            "stage_bytes": part["scan"] + part["prepass"], "step_bytes": sum(part.values()),
            "scan_traced_us": times["scan"], "stage_traced_us": times["scan"] + times["prepass"],
            "decoder_traced_us": times["decoder"], "fetch_scale": fs, "write_scale": ws}
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(res, f, indent=1)
    print(json.dumps(res))
    return 0


def event_model_bytes(U, P, C, K, H, s_a=2) -> dict:
    """Algorithmic bytes per token-head of the event ("active state") model.

    logits 2*U*P*s_a, x C*s_a, gamma s_a, y C*s_a, position 4/H, every write
    a fp32 row + mass read-modify-write, every read a fp32 row read.
    """
    op = 2 * U * P * s_a + C * s_a + s_a + C * s_a + 4.0 / H + K * (2 * C * 4 + 2 * 4) + K * C * 4
    # the segment scan itself: decoded (idx, val) pairs instead of logits
    seg = op - 2 * U * P * s_a - 4.0 / H + 2 * K * 8
    # the slot rows the scan moves through LDS (its state stays there): each
    # write loads and stores a row of C fp32, each read loads one
    lds = K * 2 * C * 4 + K * C * 4
    return {"op": op, "segment": seg, "lds_rows": lds}


def make_prefill_inputs(dev, c=C2):
    from ram_cases import projected_logits
    B, H, T, C, U, P = c["B"], c["H"], c["T"], c["C"], c["U"], c["P"]
    w, r = projected_logits(B, H, U, P, T, c["d_k"], seed=c["seed"], dtype=torch.float32)
    if c["quant"]:
        w, r = (torch.round(v / c["quant"]) * c["quant"] for v in (w, r))
    w, r = w.to(torch.bfloat16), r.to(torch.bfloat16)
    g = torch.Generator().manual_seed(c["seed"] + 100)
    x = torch.randn(B, H, T, C, generator=g).to(torch.bfloat16)
    gamma = torch.sigmoid(torch.randn(B, H, T, generator=g) + c["gamma_shift"]).to(torch.bfloat16)
    pos = torch.arange(T, dtype=torch.int32).view(1, T).expand(B, T).contiguous()
    host = dict(w=w, r=r, x=x, gamma=gamma, pos=pos)
    devd = {k: v.to(dev) for k, v in host.items()}
    return host, devd


def bench_prefill(steps, warmup, dev, c=C2):
    """A prefill config through the product path's two native stages (what the
    fused ``ram_attn_forward`` op runs): record decoder, then the segment scan."""
    import ramnet_ops  # noqa: F401
    from ramnet_ops import _native as nat
    B, H, T, C, U, P, K = c["B"], c["H"], c["T"], c["C"], c["U"], c["P"], c["K"]
    A = P ** U
    E = c["embed"]
    host, d = make_prefill_inputs(dev, c)
    slot0 = torch.zeros(B, H, A, C, device=dev)
    mass0 = torch.full((B, H, A), 1.0 / A, device=dev)
    slot = torch.empty_like(slot0)
    mass = torch.empty_like(mass0)
    y = torch.empty_like(d["x"])
    ws = torch.empty(nat.scan_workspace_bytes(B, H, T, K, K), dtype=torch.uint8, device=dev)
    code = nat.DTYPE_CODES[d["x"].dtype]
    stream = torch.cuda.current_stream(dev).cuda_stream

    def step(ev):
        ev[0].record()
        nat.call("ramnet_topk_addr_records", d["w"].data_ptr(), d["r"].data_ptr(), d["gamma"].data_ptr(), code, None,
                 E, d["pos"].data_ptr(), B, H, U, P, T, A, K, K, 0.0, 0.0, ws.data_ptr(), ws.numel(), stream)
        ev[1].record()
        nat.call("ramnet_segment_scan", d["x"].data_ptr(), code, slot0.data_ptr(), mass0.data_ptr(), slot.data_ptr(),
                 mass.data_ptr(), y.data_ptr(), B, H, T, A, C, K, K, 0, 1e-12, ws.data_ptr(), ws.numel(), stream)
        ev[2].record()

    def events(n):
        return [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(n)]

    for ev in events(warmup):
        step(ev)
    evs = events(steps)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    for ev in evs:
        step(ev)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    total_ms = evs[0][0].elapsed_time(evs[-1][2])
    ms_per_step = total_ms / steps
    dec_ms = [ev[0].elapsed_time(ev[1]) for ev in evs]
    seg_ms = [ev[1].elapsed_time(ev[2]) for ev in evs]
    step_ms = [ev[0].elapsed_time(ev[2]) for ev in evs]
    seg_avg = sum(seg_ms) / len(seg_ms)
    dec_avg = sum(dec_ms) / len(dec_ms)
    per = event_model_bytes(U, P, C, K, H)
    state_io = 2 * B * H * A * (C + 1) * 4
    n_th = B * H * T
    seg_bytes = per["segment"] * n_th + state_io
    op_bytes = per["op"] * n_th + state_io
    # compulsory HBM bytes of a step: logits, x, gamma and positions read
    # once, y written once, the zero initial state read and the final state
    # written once
    floor_bytes = (B * H * T * (2 * U * P * 2 + C * 2 + 2 + C * 2) + B * T * 4 + state_io)
    tokens = B * T
    return {
        "host": host,
        "ms_per_step": ms_per_step,
        "wall_s": wall,
        "tokens_per_s": tokens / (ms_per_step / 1e3),
        "segment_ms": seg_avg,
        "decoder_ms": dec_avg,
        "step_ms_stats": stats(step_ms),
        "segment_ms_stats": stats(seg_ms),
        "decoder_ms_stats": stats(dec_ms),
        "segment_bytes": seg_bytes,
        "lds_row_bytes": per["lds_rows"] * n_th,
        "floor_bytes": floor_bytes,
        "op_bytes": op_bytes,
        "op_roofline_frac": (op_bytes / (ms_per_step / 1e3)) / (HBM_PEAK_GBS * 1e9),
        "bytes_per_token_head": per,
    }


def bench_train(steps, warmup, dev, c=C2):
    """One training step of the operator at a prefill config: the
    differentiable forward (decoder ops ``topk_addr_forward`` +
    ``topk_segment_forward_saved``, which keeps the rows its backward needs)
    and its backward (``topk_segment_backward_saved`` + ``topk_addr_backward``),
    the op sequence autograd runs for ``random_access_memory_attention`` at
    this shape (the recompute pair ``topk_segment_forward`` /
    ``topk_segment_backward`` where the saved pair does not apply).
    Gradients of y come in as N(0,1) bf16; the final-state gradients are zero
    (None)."""
    import ramnet_ops  # noqa: F401
    from ramnet_ops import _native as nat
    ops = torch.ops.ramnet_ops
    B, H, T, C, U, P, K = c["B"], c["H"], c["T"], c["C"], c["U"], c["P"], c["K"]
    A = P ** U
    E = c["embed"]
    _, d = make_prefill_inputs(dev, c)
    slot0 = torch.zeros(B, H, A, C, device=dev)
    mass0 = torch.full((B, H, A), 1.0 / A, device=dev)
    g = torch.Generator().manual_seed(c["seed"] + 200)
    dy = torch.randn(B, H, T, C, generator=g).to(torch.bfloat16).to(dev)
    shape = [B, H, U, P, A, T]

    saved_pair = nat.segment_saved_bytes(B, H, T, A, C, K, K, d["x"].dtype) >= 0

    def step(ev):
        ev[0].record()
        idx, val = ops.topk_addr_forward(d["w"], d["r"], E, A, d["pos"], K, K, 0.0, 0.0)
        ev[1].record()
        if saved_pair:
            saved = ops.topk_segment_forward_saved(idx, val, d["x"], d["gamma"], slot0, mass0, None, K, K, False,
                                                   1e-12)[3]
            ev[2].record()
            dval = ops.topk_segment_backward_saved(val, d["x"], d["gamma"], slot0, mass0, saved, dy, None, None, K,
                                                   K, False, 1e-12)[0]
            del saved
        else:
            ops.topk_segment_forward(idx, val, d["x"], d["gamma"], slot0, mass0, None, K, K, False, 1e-12)
            ev[2].record()
            dval = ops.topk_segment_backward(idx, val, d["x"], d["gamma"], slot0, mass0, None, dy, None, None, K, K,
                                             False, 1e-12)[0]
        ev[3].record()
        ops.topk_addr_backward(idx, val, d["w"], d["r"], dval, E, d["pos"], K, K, 0.0, 0.0, shape, d["w"].dtype)
        ev[4].record()

    def events(n):
        return [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(n)]

    for ev in events(warmup):
        step(ev)
    evs = events(steps)
    torch.cuda.synchronize()
    for ev in evs:
        step(ev)
    torch.cuda.synchronize()
    ms = evs[0][0].elapsed_time(evs[-1][4]) / steps
    stage = [sum(ev[i].elapsed_time(ev[i + 1]) for ev in evs) / steps for i in range(4)]
    return {
        "workload": f"config {c.get('name', 2)} training step of the operator: decoder + segment forward, segment "
                    f"backward + decoder backward; B={B}, H={H}, T={T}, d_v={C}, A={A}, K={K}, bf16 activations, "
                    "gradient of y ~ N(0,1), none on the final state",
        "segment_pair": "saved rows (topk_segment_forward_saved / topk_segment_backward_saved)" if saved_pair
                        else "recompute (topk_segment_forward / topk_segment_backward)",
        "ms_per_step": ms,
        "tokens_per_s": B * T / (ms / 1e3),
        "decoder_forward_ms": stage[0],
        "segment_forward_ms": stage[1],
        "segment_backward_ms": stage[2],
        "decoder_backward_ms": stage[3],
    }


def stats(vals) -> dict:
    """Median, min, max and mean of a list of timings."""
    v = sorted(vals)
    return {"median": v[len(v) // 2], "min": v[0], "max": v[-1], "mean": sum(v) / len(v), "n": len(v)}


def bench_decode(n_steps, dev, graph=True, reps=5):
    """Config 3: n_steps consecutive decode steps on the persistent state, two
    ways. The primary figure captures one ``topk_autoregressive_`` launch per
    step in a HIP graph and replays it. The labelled multi-step variant runs
    the same steps through ``topk_autoregressive_steps_``: one persistent
    launch in which each (b, h) walks all steps (it needs every step's inputs
    up front, which a serving loop does not have)."""
    import ramnet_ops  # noqa: F401
    ops = torch.ops.ramnet_ops
    c = C3
    B, H, C, U, P, K = c["B"], c["H"], c["C"], c["U"], c["P"], c["K"]
    A = P ** U
    E = H // 2
    g = torch.Generator(device=dev).manual_seed(c["seed"])
    slot = 0.5 * torch.randn(B, H, A, C, device=dev, generator=g)
    mass = torch.full((B, H, A), 1.0 / A, device=dev)
    d_k = 128
    W = torch.randn(H, d_k, U * P, device=dev, generator=g) / d_k ** 0.5
    q = torch.randn(n_steps, 2, B, H, d_k, device=dev, generator=g)
    lg = (torch.einsum('sqbhd,hdn->sqbhn', q, W) / U ** 0.5).to(torch.bfloat16).view(n_steps, 2, B, H, U, P)
    w_all, r_all = lg[:, 0].contiguous(), lg[:, 1].contiguous()
    x_all = torch.randn(n_steps, B, H, C, device=dev, generator=g).to(torch.bfloat16)
    g_all = torch.sigmoid(torch.randn(n_steps, B, H, device=dev, generator=g)).to(torch.bfloat16)
    t0 = torch.randint(0, 8192, (B,), device=dev, generator=g)
    pos_all = (t0.view(1, B) + torch.arange(n_steps, device=dev).view(n_steps, 1)).to(torch.int32).contiguous()
    no_mask = torch.empty(0, dtype=torch.bool, device=dev)
    # the CPU baseline's sample (first 16 sequences, first 32 steps, in the
    # oracle's (B, H, ..., T) layout), copied before any step changes the state
    ns, nb = min(32, n_steps), min(16, B)
    host = {"w": w_all[:ns, :nb].permute(1, 2, 3, 4, 0).cpu(), "r": r_all[:ns, :nb].permute(1, 2, 3, 4, 0).cpu(),
            "x": x_all[:ns, :nb].permute(1, 2, 0, 3).cpu(), "gamma": g_all[:ns, :nb].permute(1, 2, 0).cpu(),
            "pos": pos_all[:ns, :nb].t().long().cpu(), "slot": slot[:nb].cpu(), "mass": mass[:nb].cpu()}
    keep = []

    def run_all():
        keep.clear()
        for s in range(n_steps):
            keep.append(ops.topk_autoregressive_(w_all[s], r_all[s], x_all[s], g_all[s], slot, mass, no_mask, E,
                                                 pos_all[s], K, K, 0.0, 0.0, False, 1e-12))

    mode = "eager"
    runner = run_all
    if graph:
        try:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                run_all()  # warm-up on the capture stream
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                run_all()
            torch.cuda.synchronize()
            gr.replay()
            torch.cuda.synchronize()
            runner = gr.replay
            mode = "hip-graph"
        except Exception as exc:  # capture unsupported: fall back to eager launches, reported as such
            log(f"graph capture failed ({exc}); timing eager launches")
    runner()
    torch.cuda.synchronize()

    def timed(fn):
        out = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            out.append(e0.elapsed_time(e1) * 1e3 / n_steps)  # us per step
        return out

    per_graph = timed(runner)

    def persistent():
        ops.topk_autoregressive_steps_(w_all, r_all, x_all, g_all, slot, mass, no_mask, E, pos_all, K, K, 0.0, 0.0,
                                       False, 1e-12)

    persistent()
    torch.cuda.synchronize()
    per_multi = timed(persistent)
    bytes_step = event_model_bytes(U, P, C, K, H)["op"] * B * H
    us_g, us_m = stats(per_graph), stats(per_multi)
    frac = lambda us: (bytes_step / (us * 1e-6)) / (HBM_PEAK_GBS * 1e9)
    out = {
        "host": host,
        "mode": mode,
        "steps": n_steps,
        "ms_per_step": us_g["median"] / 1e3,
        "us_per_step": us_g,
        "tokens_per_s": B / (us_g["median"] * 1e-6),
        "bytes_per_step": bytes_step,
        "roofline_frac": frac(us_g["median"]),
        "multi_step": {
            "variant": "labelled multi-step persistent launch (topk_autoregressive_steps_): all steps' inputs "
                       "given up front, one launch for the whole sequence",
            "us_per_step": us_m,
            "tokens_per_s": B / (us_m["median"] * 1e-6),
            "achieved_gbs": bytes_step / (us_m["median"] * 1e-6) / 1e9,
            "roofline_frac": frac(us_m["median"]),
        },
    }
    if mode == "hip-graph":
        out["graph_node_floor_us"] = graph_node_floor_us(dev, n_steps)
    return out


def graph_node_floor_us(dev, n_nodes):
    """Per-node time of a captured graph of n_nodes trivial kernels (an
    in-place add on 64 floats): the launch floor under one decode step."""
    x = torch.zeros(64, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        x.add_(1.0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        for _ in range(n_nodes):
            x.add_(1.0)
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        gr.replay()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / n_nodes)
    return best


def bench_lm(dev, new_tokens):
    """Config 5 through the caller harness (``ramnet_harness``): one prefill of
    the prompt with fresh states, then greedy decode steps captured as one HIP
    graph per step (model forward + in-place state update + argmax), replayed."""
    from ramnet_harness import HarnessConfig, RamLM
    c = C5
    cfg = HarnessConfig(vocab=c["vocab"], layers=c["layers"], d_model=c["d_model"], heads=c["heads"],
                        value_chs=c["C"], addr_order=c["U"], addr_radix=c["P"], top_k=c["K"], embed_num=c["embed"],
                        mlp_width=c["mlp"], dtype=torch.bfloat16)
    torch.manual_seed(c["seed"])
    model = RamLM(cfg)
    model.init_weights()
    model = model.to(device=dev, dtype=torch.bfloat16).eval()
    B, T = c["B"], c["T"]
    g = torch.Generator(device=dev).manual_seed(c["seed"])
    prompt = torch.randint(0, c["vocab"], (B, T), device=dev, generator=g)
    pos = torch.arange(T, device=dev).view(1, T).expand(B, T)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.no_grad():
        model(prompt[:, :256], model.fresh_state(B, dev), pos[:, :256], inplace=False)  # library warm-up
        states = model.fresh_state(B, dev)
        torch.cuda.synchronize()
        e0.record()
        logits, states = model(prompt, states, pos, inplace=False)
        e1.record()
        torch.cuda.synchronize()
        prefill_ms = e0.elapsed_time(e1)
        tok = logits[:, -1].argmax(-1, keepdim=True)
        p = torch.full((B, 1), T, device=dev, dtype=torch.long)

        def step():
            lg, _ = model(tok, states, p, inplace=True)
            tok.copy_(lg[:, -1].argmax(-1, keepdim=True))
            p.add_(1)

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()  # warm-up on the capture stream
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        torch.cuda.synchronize()
        n = max(1, new_tokens - 2)
        e0.record()
        for _ in range(n):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        step_ms = e0.elapsed_time(e1) / n
    finite = all(bool(torch.isfinite(sl).all()) for sl, _ in states)
    return {
        "workload": f"config 5 harness: {c['layers']} blocks, d_model={c['d_model']}, H={c['heads']}, d_v={c['C']}, "
                    f"A={c['P'] ** c['U']} (U={c['U']}, P={c['P']}), K={c['K']}, vocab={c['vocab']}, SwiGLU width "
                    f"{c['mlp']}, bf16 weights (random init), prompt {B} x {T}, {new_tokens} greedy tokens",
        "prefill_ms": prefill_ms,
        "prefill_tokens_per_s": B * T / (prefill_ms / 1e3),
        "decode_ms_per_step": step_ms,
        "decode_tokens_per_s": B / (step_ms / 1e3),
        "decode_mode": "hip-graph per step",
        "state_finite": finite,
    }


def cpu_model() -> str:
    """The host CPU's model string (/proc/cpuinfo), or the platform's name."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _cpu_threads() -> int:
    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    return n


def _dense(w, r, x, gm, slot, mass, E, pos, K, chunk=256):
    """One timed run of the oracle's dense restatement of the reference
    algorithm (torch_impl.py:217-288): dense decode of all slots, then the
    per-step dense GSU."""
    import oracle
    t0 = time.perf_counter()
    oracle.dense_ram_attn(w, r, x, gm, slot, mass, None, E, pos, (K, K), (0.0, 0.0), False, 1e-12, chunk=chunk)
    return time.perf_counter() - t0


def cpu_baseline(host, c=C2, target_s=12.0, min_tokens=512, name="config 2"):
    """Dense reference algorithm (oracle restatement) on host cores over a
    bounded sample of a prefill config's inputs: the first ``min_tokens``
    tokens (or more, up to ``target_s`` seconds) of as many batch rows as fit
    the time budget (at least one). A 16-token run of one row calibrates."""
    n = _cpu_threads()
    H, C, U, P, K, T, B = c["H"], c["C"], c["U"], c["P"], c["K"], c["T"], c["B"]
    A = P ** U

    def run(rows, tokens):
        sl = (slice(0, rows), Ellipsis, slice(0, tokens))
        return _dense(host["w"][sl], host["r"][sl], host["x"][:rows, :, :tokens], host["gamma"][:rows, :, :tokens],
                      torch.zeros(rows, H, A, C), torch.full((rows, H, A), 1.0 / A), c["embed"],
                      host["pos"][:rows, :tokens].long(), K)

    cal = max(run(1, 16), 1e-3) / 16  # seconds per token-row
    rows = int(max(1, min(B, target_s / (cal * min_tokens))))
    tokens = int(min(T, max(min_tokens, target_s / (cal * rows))))
    tokens = max(16, (tokens // 16) * 16)
    dt = run(rows, tokens)
    return {
        "value": rows * tokens / dt,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{name} inputs: {rows} of {B} batch rows x first {tokens} of {T} tokens, all {H} heads; dense "
                  f"decode of all {A} slots + per-step dense GSU (the reference torch_impl.py algorithm), "
                  f"{dt:.1f} s",
        "cpu": cpu_model(),
        "seconds": dt,
    }


def cpu_baseline_c1():
    """Config 1 in full (B=1, H=4, T=256, d_k=d_v=64, U=2, P=16, K=4, fp32,
    CAPE on 2 heads, zero state): one warm-up run, then the timed run."""
    from ram_cases import projected_logits
    n = _cpu_threads()
    B, H, T, C, U, P, K = 1, 4, 256, 64, 2, 16, 4
    A = P ** U
    w, r = projected_logits(B, H, U, P, T, 64, seed=1, dtype=torch.float32)
    g = torch.Generator().manual_seed(101)
    x = torch.randn(B, H, T, C, generator=g)
    gm = torch.sigmoid(torch.randn(B, H, T, generator=g))
    pos = torch.arange(T).view(1, T)
    args = (w, r, x, gm, torch.zeros(B, H, A, C), torch.full((B, H, A), 1.0 / A), 2, pos, K)
    _dense(*args, chunk=64)
    dt = _dense(*args, chunk=64)
    return {"value": B * T / dt, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"config 1 in full: B={B}, H={H}, T={T}, d_v={C}, A={A}, K={K}, fp32, {dt:.2f} s",
            "cpu": cpu_model(), "seconds": dt}


def cpu_baseline_c3(host, target_s=10.0, steps=32):
    """Config 3: ``steps`` consecutive decode steps from the persistent state
    (the dense restatement walks them in order, one dense GSU per step) for as
    many batch rows as fit the time budget; one step of one row calibrates."""
    n = _cpu_threads()
    c = C3
    H, C, U, P, K, B = c["H"], c["C"], c["U"], c["P"], c["K"], c["B"]
    A = P ** U
    rows_max = host["slot"].shape[0]
    steps = min(steps, host["w"].shape[-1])

    def run(rows, t):
        return _dense(host["w"][:rows, ..., :t], host["r"][:rows, ..., :t], host["x"][:rows, :, :t],
                      host["gamma"][:rows, :, :t], host["slot"][:rows].clone(), host["mass"][:rows].clone(),
                      H // 2, host["pos"][:rows, :t], K, chunk=t)

    cal = max(run(1, 1), 1e-3)  # seconds per row-step
    rows = int(max(1, min(rows_max, target_s / (cal * steps))))
    dt = run(rows, steps)
    return {"value": rows * steps / dt, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"config 3: {rows} of {B} sequences x {steps} consecutive decode steps, all {H} heads on the "
                      f"{A}x{C} fp32 state per head (dense decode + per-step dense GSU), {dt:.1f} s",
            "cpu": cpu_model(), "seconds": dt}


def bench_c1(dev, reps=20):
    """Config 1 on the GPU: the fused forward (decoders + scan) of the whole
    sequence, fp32, through the public API's native op."""
    import ramnet_ops  # noqa: F401
    from ram_cases import projected_logits
    ops = torch.ops.ramnet_ops
    B, H, T, C, U, P, K = 1, 4, 256, 64, 2, 16, 4
    A = P ** U
    w, r = projected_logits(B, H, U, P, T, 64, seed=1, dtype=torch.float32, device=dev)
    g = torch.Generator().manual_seed(101)
    x = torch.randn(B, H, T, C, generator=g).to(dev)
    gm = torch.sigmoid(torch.randn(B, H, T, generator=g)).to(dev)
    pos = torch.arange(T, dtype=torch.int32, device=dev).view(1, T)
    slot = torch.zeros(B, H, A, C, device=dev)
    mass = torch.full((B, H, A), 1.0 / A, device=dev)
    f = lambda: ops.ram_attn_forward(w, r, x, gm, slot, mass, None, 2, pos, K, K, 0.0, 0.0, False, 1e-12)
    f()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        f()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    st = stats(ts)
    return {"workload": f"config 1: B={B}, H={H}, T={T}, d_v={C}, U={U}, P={P} (A={A}), K={K}, fp32, CAPE on 2 "
                        "heads, one fused forward call (latency-bound)",
            "ms_per_call": st, "tokens_per_s": B * T / (st["median"] / 1e3)}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--decode-steps", type=int, default=C3["steps"])
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="CPU time budget per baseline (config 2; configs 3 and 4 take 3/4 of it)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--only", choices=("prefill", "decode", "stress", "lm", "train"), default=None)
    ap.add_argument("--no-train", action="store_true", help="skip the config-2 training-step line")
    ap.add_argument("--no-lm", action="store_true", help="skip the config-5 model harness line")
    ap.add_argument("--lm-tokens", type=int, default=C5["new"])
    ap.add_argument("--no-stress", action="store_true", help="skip the config-4 stress prefill lines")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB")
    ap.add_argument("--traffic-summary", default=None, metavar="DIR",
                    help="write the counter-measured traffic file from rocprofv3 runs in DIR, then exit")
    args = ap.parse_args(argv)
    if args.traffic_summary:
        return traffic_summary(args.traffic_summary)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU only: the operator shards over (batch, head) "
                                   "with no communication, so a multi-GPU figure is N independent copies of the "
                                   "one-GPU run; use --gpus 1"}), flush=True)
        return 2
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP device visible"}), flush=True)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.copy_probe > 0:
        n = args.copy_probe * (1 << 20) // 4
        src = torch.ones(n, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: {args.copy_probe} MiB read + {args.copy_probe} MiB written")
        del src, dst

    out = {"metric": METRIC}
    pre = dec = None
    if args.only in (None, "prefill"):
        log("prefill: building config 2 inputs")
        pre = bench_prefill(args.steps, args.warmup, dev)
        log(f"prefill: {pre['ms_per_step']:.3f} ms/step, segment {pre['segment_ms']:.3f} ms, "
            f"decoder {pre['decoder_ms']:.3f} ms")
    traffic = load_traffic()
    stress = {}
    stress_host = None
    if args.only == "stress" or (args.only is None and not args.no_stress):
        for name, c in (("config4", C4), ("config4_tie_heavy", C4_TIES)):
            log(f"stress: {name} prefill")
            st = bench_prefill(max(3, args.steps // 4), 1, dev, c)
            host_c4 = st.pop("host")
            if name == "config4":
                stress_host = host_c4
            seg_gbs = st["segment_bytes"] / (st["segment_ms"] / 1e3) / 1e9
            stress[name] = {
                "workload": f"B={c['B']}, H={c['H']}, T={c['T']}, d_v={c['C']}, U={c['U']}, P={c['P']} "
                            f"(A={c['P'] ** c['U']}), K={c['K']}, CAPE on {c['embed']} heads, "
                            f"gamma=sigmoid(N(0,1)), logits quantised to {c['quant']}" if c["quant"] else
                            f"B={c['B']}, H={c['H']}, T={c['T']}, d_v={c['C']}, U={c['U']}, P={c['P']} "
                            f"(A={c['P'] ** c['U']}), K={c['K']}, CAPE on {c['embed']} heads, gamma=sigmoid(N(0,1))",
                "tokens_per_s": st["tokens_per_s"], "ms_per_step": st["ms_per_step"],
                "step_ms_stats": st["step_ms_stats"], "segment_ms_stats": st["segment_ms_stats"],
                "decoder_ms": st["decoder_ms"], "segment_ms": st["segment_ms"],
                "event_model_op_frac": st["op_roofline_frac"],
                "event_model_segment_frac": seg_gbs / HBM_PEAK_GBS, "op_bytes_per_step": st["op_bytes"],
                "floor_bytes_per_step": st["floor_bytes"],
            }
            tr = traffic.get("configs", {}).get("config4") if traffic and name == "config4" else None
            if tr:
                stress[name]["hbm_counter"] = {
                    "stage_bytes": tr["stage_bytes"], "step_bytes": tr["step_bytes"],
                    "stage_gbs": tr["stage_bytes"] / (st["segment_ms"] / 1e3) / 1e9,
                    "stage_frac": tr["stage_bytes"] / (st["segment_ms"] / 1e3) / 1e9 / HBM_PEAK_GBS,
                    "step_vs_floor": tr["step_bytes"] / st["floor_bytes"], "current": traffic["current"]}
            log(f"stress: {name} {st['ms_per_step']:.3f} ms/step = {st['tokens_per_s'] / 1e6:.1f} M tokens/s, "
                f"segment {st['segment_ms']:.3f} ms, decoder {st['decoder_ms']:.3f} ms")
    train = None
    if args.only == "train" or (args.only is None and not args.no_train):
        log("train: config 2 operator forward + backward")
        train = bench_train(max(3, args.steps // 4), 1, dev)
        log(f"train: {train['ms_per_step']:.3f} ms/step = {train['tokens_per_s'] / 1e6:.2f} M tokens/s "
            f"(decoder fwd {train['decoder_forward_ms']:.3f}, segment fwd {train['segment_forward_ms']:.3f}, "
            f"segment bwd {train['segment_backward_ms']:.3f}, decoder bwd {train['decoder_backward_ms']:.3f} ms)")
    if args.only in (None, "decode"):
        log("decode: config 3, graph-captured steps")
        dec = bench_decode(args.decode_steps, dev, graph=not args.no_graph)
        log(f"decode: {dec['ms_per_step'] * 1e3:.2f} us/step ({dec['mode']}), graph node floor "
            f"{dec.get('graph_node_floor_us', float('nan')):.2f} us; multi-step launch "
            f"{dec['multi_step']['us_per_step']['median']:.2f} us/step "
            f"({dec['multi_step']['roofline_frac'] * 100:.0f}% of HBM peak)")
    c1 = None
    if args.only is None:
        log("config 1: fused forward, fp32")
        c1 = bench_c1(dev)
        log(f"config 1: {c1['ms_per_call']['median']:.3f} ms per call")

    if pre is not None:
        seg_s = pre["segment_ms"] / 1e3
        event_gbs = pre["segment_bytes"] / seg_s / 1e9
        tr = traffic["configs"]["config2"] if traffic else None
        hbm_bytes = tr["stage_bytes"] if tr else None
        hbm_gbs = None if tr is None else hbm_bytes / seg_s / 1e9
        lds_peak = lds_read_peak(dev)
        lds_gbs = pre["lds_row_bytes"] / seg_s / 1e9
        out.update({
            "value": pre["tokens_per_s"],
            "unit": "tokens/s",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": pre["ms_per_step"],
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "f32",
            "data": "synthetic",
            "config": {
                "workload": "config 2 segment-parallel prefill: B=8, H=16, T=4096, d_v=128, U=2, P=32 (A=1024), "
                            "K=8 write + 8 read, CAPE on 8 of 16 heads, gamma=sigmoid(N(0,1)-1), zero initial "
                            "state; logits = (q ~ N(0,1), d_k=128) @ W / sqrt(U)",
                "activations": "bf16", "state": "f32", "tokens_per_step": C2["B"] * C2["T"],
                "segment_length": 128,
            },
            "roofline": {
                # The dominant stage is the segment stage (one C-ABI call: the
                # mass pre-pass kernels, then segment_scan_kernel), timed live
                # with HIP events. achieved / frac: its HBM bytes per call as
                # rocprofv3's FETCH_SIZE / WRITE_SIZE count them (calibrated on
                # a copy), over that time, against the HBM peak. It does not
                # bind: the slot state stays in LDS for the whole call, and
                # the scan is bound by its per-token LDS round trips ("lds"
                # below: the slot rows it moves through LDS against the LDS
                # read peak measured in this run).
                "bound": "lds",
                "peak_resource": "hbm",
                "kernel": "segment stage: mass pre-pass + segment_scan_kernel",
                "achieved": hbm_gbs,
                "peak": HBM_PEAK_GBS,
                "unit": "GB/s",
                "frac": None if hbm_gbs is None else hbm_gbs / HBM_PEAK_GBS,
                "traffic": hbm_bytes,
                "traffic_current": None if traffic is None else traffic["current"],
                "traffic_source": os.path.relpath(TRAFFIC_FILE, REPO),
                "kernel_ms": pre["segment_ms"],
                "kernel_ms_stats": pre["segment_ms_stats"],
                "event_model_bytes": pre["segment_bytes"],
                "event_model_gbs": event_gbs,
                "event_model_frac": event_gbs / HBM_PEAK_GBS,
                "lds": {
                    "row_bytes": pre["lds_row_bytes"],
                    "achieved_gbs": lds_gbs,
                    "peak_gbs": None if lds_peak is None else lds_peak["gbs"],
                    "frac": None if lds_peak is None else lds_gbs / lds_peak["gbs"],
                    "peak_probe": lds_peak,
                },
                "step_hbm": None if tr is None else {
                    "bytes": tr["step_bytes"], "floor_bytes": pre["floor_bytes"],
                    "vs_floor": tr["step_bytes"] / pre["floor_bytes"],
                    "decoder_bytes": tr["decoder_bytes"], "stage_bytes": tr["stage_bytes"]},
            },
            "prefill": {
                "tokens_per_s": pre["tokens_per_s"],
                "step_ms_stats": pre["step_ms_stats"],
                "event_model_op_frac": pre["op_roofline_frac"],
                "decoder_ms": pre["decoder_ms"],
                "segment_ms": pre["segment_ms"],
                "op_bytes_per_step": pre["op_bytes"],
                "bytes_per_token_head": pre["bytes_per_token_head"],
            },
        })
    dec_host = None
    if dec is not None:
        dec_host = dec.pop("host")
        out["decode"] = dec
        if pre is None:
            out.update({"value": dec["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": dec["steps"],
                        "warmup": 1, "ms_per_step": dec["ms_per_step"], "higher_is_better": True,
                        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
                        "config": {"workload": "config 3 decode: B=64, H=16, A=1024, d_v=128, K=8, 512 steps"}})
    lm = None
    if args.only == "lm" or (args.only is None and not args.no_lm):
        log("lm: config 5 harness (prefill, then graph-captured greedy steps)")
        lm = bench_lm(dev, args.lm_tokens)
        log(f"lm: prefill {lm['prefill_ms']:.1f} ms = {lm['prefill_tokens_per_s'] / 1e6:.2f} M tokens/s, "
            f"decode {lm['decode_ms_per_step']:.3f} ms/step = {lm['decode_tokens_per_s']:.0f} tokens/s")
        out["lm"] = lm
        if args.only == "lm":
            out.update({"value": lm["prefill_tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": 1,
                        "warmup": 1, "ms_per_step": lm["prefill_ms"], "higher_is_better": True, "scaling": "weak",
                        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
                        "config": {"workload": lm["workload"]}})
    if train is not None:
        out["train"] = train
        if args.only == "train":
            out.update({"value": train["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1,
                        "steps": max(3, args.steps // 4), "warmup": 1, "ms_per_step": train["ms_per_step"],
                        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
                        "data": "synthetic", "config": {"workload": train["workload"]}})
    if stress:
        out["stress"] = stress
        if pre is None and dec is None:
            st = stress["config4"]
            out.update({"value": st["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": max(3, args.steps // 4),
                        "warmup": 1, "ms_per_step": st["ms_per_step"], "higher_is_better": True, "scaling": "weak",
                        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
                        "config": {"workload": "config 4 stress prefill: " + st["workload"]}})
    if c1 is not None:
        out["config1"] = c1
    if pre is not None and not args.no_cpu_baseline:
        log("cpu baseline: dense reference algorithm on host cores (config 2)")
        out["cpu_baseline"] = cpu_baseline(pre["host"], target_s=args.cpu_seconds)
        more = {}
        if c1 is not None:
            log("cpu baseline: config 1 in full")
            more["config1"] = cpu_baseline_c1()
        if dec_host is not None:
            log("cpu baseline: config 3, 32 decode steps")
            more["config3"] = cpu_baseline_c3(dec_host, target_s=args.cpu_seconds * 0.75)
        if stress_host is not None:
            log("cpu baseline: config 4, 512 tokens")
            more["config4"] = cpu_baseline(stress_host, C4, target_s=args.cpu_seconds * 0.75, name="config 4")
        out["cpu_baselines"] = more
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

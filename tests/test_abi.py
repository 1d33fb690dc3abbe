"""The C ABI and the Python host layer, without a GPU.

* every function ``include/ramnet_hip.h`` declares is exported by the built
  library and bound (with the same arity) in ``ramnet_ops._native``;
* argument validation rejects bad calls with RAMNET_EINVAL and a message
  before anything is launched;
* the Python entry points raise the reference's error types
  (ram_attn.py:81-88,298-320; cuda_impl.py:187-195; tests at
  test_cuda_address.py:108-126) and never fall back to a CPU computation.
"""
from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "ramnet_hip.h")


def _native():
    from ramnet_ops import _native
    return _native


def _declared():
    """name -> number of parameters, for every function in the header."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ramnet_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else len(params.split(","))
    return out


def test_header_declares_the_operator_entry_points():
    names = set(_declared())
    for required in ("ramnet_abi_version", "ramnet_int_bits", "ramnet_last_error", "ramnet_topk_addr_single_forward",
                     "ramnet_topk_addr_forward", "ramnet_topk_segment_forward", "ramnet_topk_segment_forward_",
                     "ramnet_topk_autoregressive_", "ramnet_ram_attn_forward", "ramnet_scan_workspace_bytes64"):
        assert required in names, required


def test_library_exports_every_declared_symbol():
    nat = _native()
    handle = ctypes.CDLL(nat.LIB_PATH)
    for name, arity in _declared().items():
        assert hasattr(handle, name), f"{name} declared in ramnet_hip.h but not exported"
        assert name in nat.SIGNATURES, f"{name} not bound in _native.SIGNATURES"
        assert len(nat.SIGNATURES[name][1]) == arity, f"{name}: header has {arity} parameters"
    assert set(nat.SIGNATURES) <= set(_declared()), "binding for a function the header does not declare"


def test_version_and_index_width():
    lib = _native().lib()
    text = open(HEADER).read()
    assert lib.ramnet_abi_version() == int(re.search(r"#define RAMNET_ABI_VERSION (\d+)", text).group(1))
    assert lib.ramnet_int_bits() == 32


def test_workspace_size_formula():
    lib = _native().lib()
    for B, H, T, kw, kr in ((8, 16, 4096, 8, 8), (1, 1, 1, 1, 1), (2, 3, 33, 4, 12), (1, 2, 0, 3, 3)):
        t_pad = (T + 31) // 32 * 32
        # write records (16 B) and read records (8 B), then one 16-byte gain
        # record per (event, token) for the precomputed-gain scan, then one
        # int of read-after-write flags per token for the paired scan
        want = B * H * t_pad * (kw * 16 + kr * 8) + B * H * t_pad * max(kw, kr) * 16 + B * H * t_pad * 4
        assert lib.ramnet_scan_workspace_bytes64(B, H, T, kw, kr) == want
    assert lib.ramnet_scan_workspace_bytes(1 << 20, 64, 1 << 20, 8, 8) == -1  # > int32


FAKE = 0x1000  # never dereferenced: every call below fails validation first


def _einval(fn, *args, match):
    nat = _native()
    rc = getattr(nat.lib(), fn)(*args)
    assert rc == nat.RAMNET_EINVAL, f"{fn} returned {rc}"
    msg = nat.lib().ramnet_last_error().decode()
    assert re.search(match, msg), msg
    with pytest.raises(RuntimeError, match=match):
        nat.call(fn, *args)


def test_decoder_argument_checks():
    f = "ramnet_topk_addr_single_forward"
    ok = dict(addr=FAKE, dtype=2, B=1, H=2, U=2, P=4, T=8, E=1, A=16, pos=FAKE, k=4, r=0.0, neg=0, enc=1, idx=FAKE,
              val=FAKE, stream=None)

    def call(match, **kw):
        a = {**ok, **kw}
        _einval(f, *a.values(), match=match)
    call("address shape", B=-1)
    call("address shape", U=0)
    call("A must equal P", A=15)
    call("Address space overflow", U=31, P=2, A=1 << 31)
    call("embed_num", E=3)
    call("dtype", dtype=7)
    call("top_k", k=17)
    call("top_k", k=0)
    call("top_k_re_norm", r=1.5)
    call("null tensor pointer", addr=None)
    call("index overflow", B=1 << 20, T=1 << 12)


def test_segment_and_decode_argument_checks():
    seg = "ramnet_topk_segment_forward"
    # idx, val, x, gamma, dtype, mask, init_slot, init_mass, slot_out, mass_out, y, B, H, T, A, C, kw, kr,
    # mass_aware, eps, workspace, bytes, stream
    base = [FAKE, FAKE, FAKE, FAKE, 2, None, FAKE, FAKE + 256, FAKE, FAKE + 512, FAKE, 1, 2, 8, 16, 4, 4, 4, 0, 1e-12,
            FAKE, 1 << 20, None]
    _einval(seg, *base[:19], 0.0, *base[20:], match="eps")
    _einval(seg, *base[:16], 17, *base[17:], match="top_k")
    bad_alias = list(base)
    bad_alias[9] = bad_alias[7]  # mass_out == init_mass
    _einval(seg, *bad_alias, match="must not alias")
    small = list(base)
    small[21] = 16
    _einval(seg, *small, match="workspace too small")
    dec = "ramnet_topk_autoregressive_"
    args = [FAKE, FAKE, FAKE, FAKE, 2, FAKE, FAKE, None, 1, FAKE, 1, 2, 2, 4, 16, 8, 4, 4, 0.0, 0.0, 0, 1e-12,
            FAKE, None]
    _einval(dec, *args[:14], 15, *args[15:], match="A must equal P|A ")
    _einval(dec, *args[:21], 0.0, *args[22:], match="eps")
    _einval(dec, *args[:4], 9, *args[5:], match="dtype")


# ---- Python host layer (reference error types; no CPU fallback)

def _small_inputs(device="cpu", T=5, H=2, U=2, P=4, C=8):
    w = torch.randn(1, T, H, U, P, device=device)
    return w, w.clone(), torch.randn(1, T, H, C, device=device)


def test_api_type_and_value_errors():
    from ramnet_ops import random_access_memory_attention as ram, topk_addr
    w, r, v = _small_inputs()
    with pytest.raises(TypeError):
        ram(w, r, v, top_k=2.5)
    with pytest.raises(TypeError):
        ram(w, r, v, top_k=(1, 2, 3))
    with pytest.raises(ValueError):
        ram(w, r, v, top_k_re_norm=1.5)
    with pytest.raises(TypeError):
        ram(w, r, v, top_k_re_norm="x")
    with pytest.raises(ValueError):
        ram(w, r, v, impl_backend="nope")
    with pytest.raises(AssertionError, match="top_k"):
        ram(w, r, v, top_k=17)
    addr = torch.randn(1, 2, 2, 4, 5)
    with pytest.raises(ValueError):
        topk_addr(addr, 0, torch.zeros(1, 5, dtype=torch.long), 4, 2.0)
    with pytest.raises(TypeError):
        topk_addr(addr, 0, torch.zeros(1, 5, dtype=torch.long), 4, None)


def test_api_has_no_cpu_fallback():
    from ramnet_ops import random_access_memory_attention as ram, topk_addr
    w, r, v = _small_inputs()
    with pytest.raises(RuntimeError, match="not part of this package"):
        ram(w, r, v, impl_backend="torch")
    with pytest.raises(RuntimeError):
        ram(w, r, v)  # CPU tensors: the HIP path refuses them
    with pytest.raises(RuntimeError):
        topk_addr(torch.randn(1, 2, 2, 4, 5), 0, torch.zeros(1, 5, dtype=torch.long), 4, 0.0)


def test_cuda_path_capacity_asserts():
    """Address-space and int32-capacity checks fire before any launch
    (reference test_cuda_address.py:108-126), here on meta tensors."""
    from ramnet_ops.impl.cuda_impl import _cuda_ram_attn
    m = torch.device("meta")

    def run(B, H, U, P, T, C):
        A = P ** U
        w = torch.empty(B, H, U, P, T, device=m)
        x = torch.empty(B, H, T, C, device=m)
        _cuda_ram_attn(w, w, x, torch.empty(B, H, T, device=m), torch.empty(B, H, A, C, device=m),
                       torch.empty(B, H, A, device=m), None, 0, torch.empty(B, T, dtype=torch.long, device=m),
                       (1, 1), (0.0, 0.0), False, 1e-12, False)
    with pytest.raises(AssertionError, match="Address space overflow"):
        run(1, 1, 31, 2, 2, 4)
    with pytest.raises(AssertionError, match="CUDA index overflow"):
        run(64, 64, 2, 64, 4, 256)


def test_scan_plan_envelope():
    """The scan planner (``ramnet_segment_plan``, no device work) accepts every
    shape up to A = 8190 slots and top-K 128 with an LDS footprint within the
    160 KiB of a CU; wider slot spaces in the precomputed-gain form (split
    into slot ranges), as far as the int32 limit B*H*A*C < 2**31 allows; it
    refuses top-K beyond 128 and shapes past the int32 limits."""
    from ramnet_ops import _native as nat
    for A in (4, 16, 256, 1024, 2401, 4096, 6561, 8100, 8190):
        for C in (1, 7, 16, 100, 128, 512):
            for K in (1, 8, 16, 64, 100, 128):
                for dtype in (torch.float32, torch.bfloat16):
                    plan = nat.segment_plan(8, 16, A, C, K, K, dtype)
                    assert plan is not None, (A, C, K, dtype)
                    cs, lds, _ = plan
                    assert 1 <= cs and 0 < lds <= 160 * 1024, (A, C, K, cs, lds)
    for A in (8192, 16384, 32768, 40958, 40960, 65536, 1 << 17):
        for C, K in ((128, 8), (7, 64), (256, 128)):
            B = max(1, min(8, (2 ** 31 - 1) // (16 * A * C)))
            plan = nat.segment_plan(B, 16, A, C, K, K)
            assert plan is not None and plan[2], (A, C, K, plan)
            assert 0 < plan[1] <= 160 * 1024, (A, plan)
    assert nat.segment_plan(1, 1, 1 << 20, 16, 8, 8) is not None
    assert nat.segment_plan(8, 16, 1024, 128, 8, 129) is None
    assert nat.segment_plan(8, 16, 1 << 20, 128, 8, 8) is None  # B*H*A*C beyond int32
    assert nat.segment_plan(8, 16, 1024, 128, 4, 12) is not None  # Kw != Kr
    assert nat.segment_plan(0, 16, 1024, 128, 8, 8) is None


def test_segment_workspace_query():
    """``ramnet_segment_workspace_bytes`` sizes the forward's workspace for
    the exact shape: the records and gain records of
    ``ramnet_scan_workspace_bytes`` for a slot space held in one slice; a
    scan in slot ranges with 16-bit activations adds B*H*T*C fp32 read sums
    (fp32 activations keep them in y); -1 for shapes the scan refuses."""
    from ramnet_ops import _native as nat
    for (B, H, T, A, C, K) in ((8, 16, 4096, 1024, 128, 8), (2, 3, 33, 4096, 7, 16), (1, 2, 100, 8190, 24, 64)):
        for dtype in (torch.float32, torch.float16, torch.bfloat16):
            assert nat.segment_workspace_bytes(B, H, T, A, C, K, K, dtype) == nat.scan_workspace_bytes(B, H, T, K, K)
    B, H, T, A, C, K = 1, 2, 300, 65536, 24, 8
    base = nat.scan_workspace_bytes(B, H, T, K, K)
    assert nat.segment_workspace_bytes(B, H, T, A, C, K, K, torch.float32) == base
    for dtype in (torch.float16, torch.bfloat16):
        assert nat.segment_workspace_bytes(B, H, T, A, C, K, K, dtype) == base + B * H * T * C * 4
    assert nat.segment_workspace_bytes(B, H, 0, A, C, K, K, torch.bfloat16) == nat.scan_workspace_bytes(B, H, 0, K, K)
    assert nat.segment_workspace_bytes(B, H, T, A, C, K, 129, torch.bfloat16) == -1
    assert nat.segment_workspace_bytes(8, 16, T, 1 << 20, 128, K, K, torch.bfloat16) == -1


def test_saved_pair_sizes():
    """``ramnet_segment_saved_bytes``: the scan records, the backward's
    per-event records (16 bytes per event), and two fp32 rows per
    padded event slot (x - s of each write, the row of each read) in the
    backward's channel slices, each part 256-byte aligned; -1 outside the
    pair's envelope. The saved backward's workspace holds everything the
    recompute backward's does but the records and the rows."""
    from ramnet_ops import _native as nat
    al = lambda n: (n + 255) // 256 * 256  # noqa: E731
    B, H, T, A, C, K = 8, 16, 4096, 1024, 128, 8
    t_pad = (T + 31) // 32 * 32
    rec = al(B * H * t_pad * (K * 16 + K * 8))
    aux = 2 * al(B * H * T * K * 16)
    rows = al(B * H * t_pad * K * C * 4)  # 8 event slots, 16 slices of 8 channels, padded tokens
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        assert nat.segment_saved_bytes(B, H, T, A, C, K, K, dtype) == rec + aux + 2 * rows
    # top-k 5 pads to 8 event slots
    assert nat.segment_saved_bytes(1, 2, 40, 64, 32, 5, 5, torch.float32) == \
        al(2 * 64 * (5 * 16 + 5 * 8)) + 2 * al(2 * 40 * 5 * 16) + 2 * al(2 * 64 * 8 * 32 * 4)
    assert nat.segment_saved_bytes(1, 2, 16, 64, 24, 8, 8, torch.float32) == -1  # no whole forward slices
    assert nat.segment_saved_bytes(1, 1, 13, 256, 16, 100, 70, torch.float32) == -1  # two event passes
    assert nat.segment_saved_bytes(1, 2, 16, 65536, 32, 8, 8, torch.float32) == -1  # slot ranges
    assert nat.segment_saved_bytes(1, 2, 0, 64, 32, 8, 8, torch.float32) == -1
    full = nat.segment_backward_workspace_bytes(B, H, T, A, C, K, K)
    assert nat.segment_backward_saved_workspace_bytes(B, H, T, A, C, K, K) == full - rec - rows


def test_scan_plan_follows_shape_and_override(monkeypatch):
    """The query plans for the shape it is given: the activation width enters
    the LDS footprint (the staged x rows), and a layout forced through
    RAMNET_SCAN_LAYOUT -- which the launch honours too -- is what the query
    reports, including its form; a layout that does not fit is refused."""
    from ramnet_ops import _native as nat
    monkeypatch.setenv("RAMNET_SCAN_LAYOUT", "1,8,1,4")
    f32 = nat.segment_plan(8, 16, 1024, 128, 8, 8, torch.float32)
    bf16 = nat.segment_plan(8, 16, 1024, 128, 8, 8, torch.bfloat16)
    assert f32[0] == bf16[0] and f32[1] > bf16[1]  # same slice, wider staged x
    monkeypatch.setenv("RAMNET_SCAN_LAYOUT", "1,16,1,2,1")
    cs, lds, pre = nat.segment_plan(4, 8, 4096, 128, 16, 16, torch.bfloat16)
    assert (cs, pre) == (2 * (64 // 16) * 1, True)
    monkeypatch.setenv("RAMNET_SCAN_LAYOUT", "1,8,1,4")
    cs, lds, pre = nat.segment_plan(8, 16, 1024, 128, 8, 8, torch.bfloat16)
    assert (cs, pre) == (4 * (64 // 8), False)
    monkeypatch.setenv("RAMNET_SCAN_LAYOUT", "1,8,1,4")
    assert nat.segment_plan(8, 16, 1024, 128, 16, 16, torch.bfloat16) is None  # 8 event lanes < top-K 16

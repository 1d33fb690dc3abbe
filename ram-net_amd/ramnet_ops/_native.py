"""ctypes binding of the gfx950 operator library (``_lib/libramnet_hip.so``).

The library exports the C ABI declared in ``include/ramnet_hip.h``. It links
the HIP runtime by soname, so torch is imported first: the runtime torch
already loaded is then the one the library binds to, and the stream handles
torch hands out are valid for it.

Loading never falls back to anything else: if the library is missing or
cannot be opened, :func:`lib` raises ``ImportError`` naming the build command.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (load torch's HIP runtime before the library)

LIB_NAME = "libramnet_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", LIB_NAME)

# int return codes of the C ABI
RAMNET_OK = 0
RAMNET_EINVAL = 1
RAMNET_ELAUNCH = 2

# activation dtype codes of the C ABI
DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_float = ctypes.c_float
_c_ptr = ctypes.c_void_p

# name -> argtypes, in header order
SIGNATURES: dict[str, tuple[type, list]] = {
    "ramnet_abi_version": (_c_int, []),
    "ramnet_int_bits": (_c_int, []),
    "ramnet_last_error": (ctypes.c_char_p, []),
    "ramnet_topk_addr_single_forward": (_c_int, [
        _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr,
        _c_i64, _c_float, _c_int, _c_int, _c_ptr, _c_ptr, _c_ptr]),
    "ramnet_topk_addr_forward": (_c_int, [
        _c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr,
        _c_i64, _c_i64, _c_float, _c_float, _c_int, _c_ptr, _c_ptr, _c_ptr]),
    "ramnet_topk_addr_single_backward": (_c_int, [
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr,
        _c_i64, _c_float, _c_int, _c_ptr, _c_ptr]),
    "ramnet_topk_addr_backward": (_c_int, [
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        _c_ptr, _c_i64, _c_i64, _c_float, _c_float, _c_ptr, _c_ptr, _c_ptr]),
    "ramnet_scan_workspace_bytes64": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "ramnet_scan_workspace_bytes": (_c_int, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "ramnet_segment_workspace_bytes": (_c_i64, [_c_i64] * 7 + [_c_int]),
    "ramnet_topk_segment_forward": (_c_int, [
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_float, _c_ptr, _c_i64, _c_ptr]),
    "ramnet_topk_segment_forward_": (_c_int, [
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_float, _c_ptr, _c_i64, _c_ptr]),
    "ramnet_topk_addr_records": (_c_int, [
        _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        _c_i64, _c_i64, _c_float, _c_float, _c_ptr, _c_i64, _c_ptr]),
    "ramnet_segment_scan": (_c_int, [
        _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        _c_i64, _c_int, _c_float, _c_ptr, _c_i64, _c_ptr]),
    "ramnet_ram_attn_forward": (_c_int, [
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_float, _c_float, _c_int,
        _c_float, _c_ptr, _c_i64, _c_ptr]),
    "ramnet_ram_attn_forward_noalloc": (_c_int, [
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_float, _c_float, _c_int,
        _c_float, _c_ptr]),
    "ramnet_topk_autoregressive_": (_c_int, [
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_ptr,
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_float, _c_float,
        _c_int, _c_float, _c_ptr, _c_ptr]),
    "ramnet_topk_autoregressive_steps_": (_c_int, [
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_ptr, _c_i64,
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_float, _c_float,
        _c_int, _c_float, _c_ptr, _c_ptr]),
    "ramnet_topk_segment_backward": (_c_int, [
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        _c_int, _c_float, _c_ptr, _c_i64, _c_ptr]),
    "ramnet_segment_backward_workspace_bytes": (_c_i64, [_c_i64] * 7),
    "ramnet_segment_saved_bytes": (_c_i64, [_c_i64] * 7 + [_c_int]),
    "ramnet_topk_segment_forward_save": (_c_int, [
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_float, _c_ptr, _c_i64, _c_ptr, _c_i64,
        _c_ptr]),
    "ramnet_segment_backward_saved_workspace_bytes": (_c_i64, [_c_i64] * 7),
    "ramnet_topk_segment_backward_saved": (_c_int, [
        _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        _c_int, _c_float, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr]),
    "ramnet_segment_plan": (_c_int, [
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, ctypes.POINTER(_c_int), ctypes.POINTER(_c_int),
        ctypes.POINTER(_c_int)]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library (loaded once per process)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_NAME} is not built ({LIB_PATH} missing); run `python ram-net_amd/build_hip.py`")
            try:
                handle = ctypes.CDLL(LIB_PATH)
            except OSError as exc:
                raise ImportError(f"cannot load {LIB_PATH}: {exc}") from exc
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


def call(name: str, *args) -> None:
    """Call a C-ABI entry point; a nonzero return becomes a RuntimeError."""
    rc = getattr(lib(), name)(*args)
    if rc != RAMNET_OK:
        msg = lib().ramnet_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def int_bits() -> int:
    return int(lib().ramnet_int_bits())


def segment_plan(B: int, H: int, A: int, C: int, w_top_k: int, r_top_k: int,
                 dtype: torch.dtype = torch.bfloat16) -> tuple[int, int, bool] | None:
    """(channel-slice width, LDS bytes, precomputed-gain form) of a segment-scan
    launch of this shape on the current device, or None if unsupported."""
    cs, lds, pre = _c_int(0), _c_int(0), _c_int(0)
    ok = lib().ramnet_segment_plan(B, H, A, C, w_top_k, r_top_k, DTYPE_CODES[dtype], ctypes.byref(cs),
                                   ctypes.byref(lds), ctypes.byref(pre))
    return (cs.value, lds.value, bool(pre.value)) if ok else None


def scan_workspace_bytes(B: int, H: int, T: int, w_top_k: int, r_top_k: int) -> int:
    """Device workspace (bytes) the segment scan needs for these sizes."""
    return int(lib().ramnet_scan_workspace_bytes64(B, H, T, w_top_k, r_top_k))


def segment_workspace_bytes(B: int, H: int, T: int, A: int, C: int, w_top_k: int, r_top_k: int,
                            dtype: torch.dtype) -> int:
    """Device workspace (bytes) of the segment forward entry points for this
    exact shape (-1: a shape the scan does not take)."""
    return int(lib().ramnet_segment_workspace_bytes(B, H, T, A, C, w_top_k, r_top_k, DTYPE_CODES[dtype]))


def segment_backward_workspace_bytes(B: int, H: int, T: int, A: int, C: int, w_top_k: int, r_top_k: int) -> int:
    """Device workspace (bytes) of the segment backward; -1 for shapes it does not take."""
    return int(lib().ramnet_segment_backward_workspace_bytes(B, H, T, A, C, w_top_k, r_top_k))


def segment_saved_bytes(B: int, H: int, T: int, A: int, C: int, w_top_k: int, r_top_k: int,
                        dtype: torch.dtype) -> int:
    """Bytes of the rows a training forward saves for its backward
    (ramnet_topk_segment_forward_save); -1 where that pair does not apply."""
    if dtype not in DTYPE_CODES:
        return -1
    return int(lib().ramnet_segment_saved_bytes(B, H, T, A, C, w_top_k, r_top_k, DTYPE_CODES[dtype]))


def segment_backward_saved_workspace_bytes(B: int, H: int, T: int, A: int, C: int, w_top_k: int,
                                           r_top_k: int) -> int:
    """Device workspace (bytes) of the segment backward that takes saved rows."""
    return int(lib().ramnet_segment_backward_saved_workspace_bytes(B, H, T, A, C, w_top_k, r_top_k))


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream

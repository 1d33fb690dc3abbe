"""``torch.library`` operators backed by the gfx950 C ABI.

Operator names follow the reference extension's dispatcher registrations
(packages/ramnet-ops/csrc/ram_attn_bind.cpp:22-113) so that
``torch.ops.ramnet_ops.<name>`` resolves to the MI355X kernels. Schemas of
the decoder and decode-step ops are the reference's; the segment ops drop the
event-grouping metadata (seg_idx/seg_off/seg_len/event_i) because the HIP
scan walks time in order and needs no sort, and take the decoded indices
instead. Every op allocates its outputs with torch and launches on the
current stream of the input's device; fake (meta) implementations give
output shapes for tracing.
"""
from __future__ import annotations

import torch
from torch import Tensor

from .. import _native as nat

_NS = "ramnet_ops"


def _code(t: Tensor) -> int:
    try:
        return nat.DTYPE_CODES[t.dtype]
    except KeyError:
        raise RuntimeError(f"ramnet_ops: unsupported dtype {t.dtype}; expected float32, float16 or bfloat16") from None


def _require_gpu(name: str, *tensors: Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{name}: tensors must be on a GPU (HIP) device, got {t.device}")


def _dims(op: str, name: str, t: Tensor, n: int) -> tuple[int, ...]:
    """The sizes of a tensor argument that must have ``n`` dimensions."""
    if not isinstance(t, Tensor):
        raise RuntimeError(f"{op}: {name} must be a tensor, got {type(t).__name__}")
    if t.dim() != n:
        raise RuntimeError(f"{op}: Tensor {name} must have {n} dimensions, but got shape {tuple(t.shape)}")
    return tuple(t.shape)


def _check_shapes(op: str, **named: tuple[Tensor | None, tuple[int, ...]]) -> None:
    """Exact sizes of every tensor argument, checked before any launch, as the
    reference's native checks do (check_tensor, csrc/cuda_utils.cuh:375-391;
    e.g. ram_attn_topk_autoregressive.cu:216-224). The kernels index every
    tensor with sizes taken from the leading ones, so a mis-shaped tensor
    raises RuntimeError here instead of reaching device memory. ``None``
    entries are optional tensors that were not given."""
    for name, (t, shape) in named.items():
        if t is None:
            continue
        if not isinstance(t, Tensor):
            raise RuntimeError(f"{op}: {name} must be a tensor, got {type(t).__name__}")
        if tuple(t.shape) != tuple(shape):
            raise RuntimeError(f"{op}: Tensor {name} shape mismatch: expect {tuple(shape)}, but got {tuple(t.shape)}")


def _check_slots(op: str, U: int, P: int, A: int) -> None:
    if P ** U != A:
        raise RuntimeError(f"{op}: the slot count A={A} must equal P**U = {P}**{U}")


def _check_decode_dtypes(op: str, w_addr: Tensor, r_addr: Tensor, x: Tensor) -> None:
    """The decode kernels read the logits in x's dtype, as the reference
    requires (check_address with x's scalar type,
    ram_attn_topk_autoregressive.cu:32-34,216): logits of another dtype
    raise RuntimeError before any launch."""
    _code(x)
    for name, t in (("w_addr", w_addr), ("r_addr", r_addr)):
        if t.dtype != x.dtype:
            raise RuntimeError(f"{op}: Tensor {name} dtype mismatch: expect {x.dtype}, but got {t.dtype}")


def _require_given(name: str, **tensors: Tensor) -> None:
    """Required tensor arguments (the dispatcher passes None through to a
    Python operator); the reference's native checks raise RuntimeError."""
    for arg, t in tensors.items():
        if not isinstance(t, Tensor):
            raise RuntimeError(f"{name}: {arg} must be a tensor, got {type(t).__name__}")


# --------------------------------------------------------------------------
# address decoder

@torch.library.custom_op(f"{_NS}::topk_addr_single_forward", mutates_args=(), device_types="cuda")
def topk_addr_single_forward(addr: Tensor, embed_num: int, A: int, position_ids: Tensor, top_k: int,
                             top_k_re_norm: float, addr_val_neg: bool = False,
                             encode_batch_idx: bool = True) -> tuple[Tensor, Tensor]:
    op = "topk_addr_single_forward"
    _require_gpu(op, addr, position_ids)
    B, H, U, P, T = _dims(op, "addr", addr, 5)
    _check_slots(op, U, P, A)
    _check_shapes(op, position_ids=(position_ids, (B, T)))
    addr = addr.contiguous()
    pos = position_ids.to(device=addr.device, dtype=torch.int32).contiguous()
    idx = torch.empty((B, H, top_k, T), dtype=torch.int32, device=addr.device)
    val = torch.empty((B, H, top_k, T), dtype=torch.float32, device=addr.device)
    with torch.cuda.device(addr.device):
        nat.call("ramnet_topk_addr_single_forward", addr.data_ptr(), _code(addr), B, H, U, P, T, embed_num, A,
                 pos.data_ptr(), top_k, float(top_k_re_norm), int(addr_val_neg), int(encode_batch_idx),
                 idx.data_ptr(), val.data_ptr(), nat.stream_of(addr))
    return idx, val


@topk_addr_single_forward.register_fake
def _(addr, embed_num, A, position_ids, top_k, top_k_re_norm, addr_val_neg=False, encode_batch_idx=True):
    B, H, _, _, T = addr.shape
    shape = (B, H, top_k, T)
    return addr.new_empty(shape, dtype=torch.int32), addr.new_empty(shape, dtype=torch.float32)


@torch.library.custom_op(f"{_NS}::topk_addr_forward", mutates_args=(), device_types="cuda")
def topk_addr_forward(w_addr: Tensor, r_addr: Tensor, embed_num: int, A: int, position_ids: Tensor, w_top_k: int,
                      r_top_k: int, w_re_norm: float, r_re_norm: float,
                      encode_batch_idx: bool = True) -> tuple[Tensor, Tensor]:
    op = "topk_addr_forward"
    _require_gpu(op, w_addr, r_addr, position_ids)
    B, H, U, P, T = _dims(op, "w_addr", w_addr, 5)
    _check_slots(op, U, P, A)
    _check_shapes(op, r_addr=(r_addr, (B, H, U, P, T)), position_ids=(position_ids, (B, T)))
    if r_addr.dtype != w_addr.dtype:
        raise RuntimeError("topk_addr_forward: w_addr and r_addr must share shape and dtype")
    w_addr, r_addr = w_addr.contiguous(), r_addr.contiguous()
    pos = position_ids.to(device=w_addr.device, dtype=torch.int32).contiguous()
    K = w_top_k + r_top_k
    idx = torch.empty((B, H, K, T), dtype=torch.int32, device=w_addr.device)
    val = torch.empty((B, H, K, T), dtype=torch.float32, device=w_addr.device)
    with torch.cuda.device(w_addr.device):
        nat.call("ramnet_topk_addr_forward", w_addr.data_ptr(), r_addr.data_ptr(), _code(w_addr), B, H, U, P, T,
                 embed_num, A, pos.data_ptr(), w_top_k, r_top_k, float(w_re_norm), float(r_re_norm),
                 int(encode_batch_idx), idx.data_ptr(), val.data_ptr(), nat.stream_of(w_addr))
    return idx, val


@topk_addr_forward.register_fake
def _(w_addr, r_addr, embed_num, A, position_ids, w_top_k, r_top_k, w_re_norm, r_re_norm, encode_batch_idx=True):
    B, H, _, _, T = w_addr.shape
    shape = (B, H, w_top_k + r_top_k, T)
    return w_addr.new_empty(shape, dtype=torch.int32), w_addr.new_empty(shape, dtype=torch.float32)


# --------------------------------------------------------------------------
# address decoder backward (reference: ram_attn_bind.cpp:36-64 schemas,
# _cuda_autograd.py:4-180 wiring)

@torch.library.custom_op(f"{_NS}::topk_addr_single_backward", mutates_args=(), device_types="cuda")
def topk_addr_single_backward(idx: Tensor, val: Tensor, addr: Tensor, D_val: Tensor, embed_num: int,
                              position_ids: Tensor, top_k: int, top_k_re_norm: float, addr_val_neg: bool,
                              shape: list[int], dtype: torch.dtype) -> Tensor:
    _require_given("topk_addr_single_backward", idx=idx, val=val, addr=addr, D_val=D_val, position_ids=position_ids)
    op = "topk_addr_single_backward"
    _require_gpu(op, idx, val, addr, D_val, position_ids)
    B, H, U, P, A, T = shape
    _check_slots(op, U, P, A)
    ev = (B, H, top_k, T)
    _check_shapes(op, idx=(idx, ev), val=(val, ev), D_val=(D_val, ev), addr=(addr, (B, H, U, P, T)),
                  position_ids=(position_ids, (B, T)))
    addr = addr.to(dtype).contiguous()
    pos = position_ids.to(device=addr.device, dtype=torch.int32).contiguous()
    grad = torch.empty((B, H, U, P, T), dtype=dtype, device=addr.device)
    with torch.cuda.device(addr.device):
        nat.call("ramnet_topk_addr_single_backward", idx.to(torch.int32).contiguous().data_ptr(),
                 val.to(torch.float32).contiguous().data_ptr(), addr.data_ptr(),
                 D_val.to(torch.float32).contiguous().data_ptr(), _code(addr), B, H, U, P, T, embed_num, A,
                 pos.data_ptr(), top_k, float(top_k_re_norm), int(addr_val_neg), grad.data_ptr(),
                 nat.stream_of(addr))
    return grad


@topk_addr_single_backward.register_fake
def _(idx, val, addr, D_val, embed_num, position_ids, top_k, top_k_re_norm, addr_val_neg, shape, dtype):
    B, H, U, P, _, T = shape
    return val.new_empty((B, H, U, P, T), dtype=dtype)


@torch.library.custom_op(f"{_NS}::topk_addr_backward", mutates_args=(), device_types="cuda")
def topk_addr_backward(idx: Tensor, val: Tensor, w_addr: Tensor, r_addr: Tensor, D_val: Tensor, embed_num: int,
                       position_ids: Tensor, w_top_k: int, r_top_k: int, w_re_norm: float, r_re_norm: float,
                       shape: list[int], dtype: torch.dtype) -> tuple[Tensor, Tensor]:
    _require_given("topk_addr_backward", idx=idx, val=val, w_addr=w_addr, r_addr=r_addr, D_val=D_val,
                   position_ids=position_ids)
    op = "topk_addr_backward"
    _require_gpu(op, idx, val, w_addr, r_addr, D_val, position_ids)
    B, H, U, P, A, T = shape
    _check_slots(op, U, P, A)
    ev = (B, H, w_top_k + r_top_k, T)
    _check_shapes(op, idx=(idx, ev), val=(val, ev), D_val=(D_val, ev), w_addr=(w_addr, (B, H, U, P, T)),
                  r_addr=(r_addr, (B, H, U, P, T)), position_ids=(position_ids, (B, T)))
    w_addr, r_addr = w_addr.to(dtype).contiguous(), r_addr.to(dtype).contiguous()
    pos = position_ids.to(device=w_addr.device, dtype=torch.int32).contiguous()
    gw = torch.empty((B, H, U, P, T), dtype=dtype, device=w_addr.device)
    gr = torch.empty_like(gw)
    with torch.cuda.device(w_addr.device):
        nat.call("ramnet_topk_addr_backward", idx.to(torch.int32).contiguous().data_ptr(),
                 val.to(torch.float32).contiguous().data_ptr(), w_addr.data_ptr(), r_addr.data_ptr(),
                 D_val.to(torch.float32).contiguous().data_ptr(), _code(w_addr), B, H, U, P, T, embed_num, A,
                 pos.data_ptr(), w_top_k, r_top_k, float(w_re_norm), float(r_re_norm), gw.data_ptr(), gr.data_ptr(),
                 nat.stream_of(w_addr))
    return gw, gr


@topk_addr_backward.register_fake
def _(idx, val, w_addr, r_addr, D_val, embed_num, position_ids, w_top_k, r_top_k, w_re_norm, r_re_norm, shape,
      dtype):
    B, H, U, P, _, T = shape
    return val.new_empty((B, H, U, P, T), dtype=dtype), val.new_empty((B, H, U, P, T), dtype=dtype)


def _single_setup(ctx, inputs, output):
    addr, embed_num, A, position_ids, top_k, top_k_re_norm, addr_val_neg, _ = inputs
    idx, val = output
    B, H, U, P, T = addr.shape
    ctx.args = (embed_num, top_k, float(top_k_re_norm), bool(addr_val_neg), [B, H, U, P, A, T], addr.dtype)
    ctx.save_for_backward(idx, val, position_ids, addr)
    ctx.mark_non_differentiable(idx)
    ctx.set_materialize_grads(False)


def _single_backward(ctx, D_idx, D_val):
    if D_val is None:
        return (None,) * 8
    idx, val, position_ids, addr = ctx.saved_tensors
    embed_num, top_k, re_norm, neg, shape, dtype = ctx.args
    grad = topk_addr_single_backward(idx, val, addr, D_val, embed_num, position_ids, top_k, re_norm, neg, shape,
                                     dtype)
    return (grad,) + (None,) * 7


topk_addr_single_forward.register_autograd(_single_backward, setup_context=_single_setup)


def _pair_setup(ctx, inputs, output):
    w_addr, r_addr, embed_num, A, position_ids, w_top_k, r_top_k, w_re_norm, r_re_norm, _ = inputs
    idx, val = output
    B, H, U, P, T = w_addr.shape
    ctx.args = (embed_num, w_top_k, r_top_k, float(w_re_norm), float(r_re_norm), [B, H, U, P, A, T], w_addr.dtype)
    ctx.save_for_backward(idx, val, position_ids, w_addr, r_addr)
    ctx.mark_non_differentiable(idx)
    ctx.set_materialize_grads(False)


def _pair_backward(ctx, D_idx, D_val):
    if D_val is None:
        return (None,) * 10
    idx, val, position_ids, w_addr, r_addr = ctx.saved_tensors
    embed_num, w_top_k, r_top_k, w_re, r_re, shape, dtype = ctx.args
    gw, gr = topk_addr_backward(idx, val, w_addr, r_addr, D_val, embed_num, position_ids, w_top_k, r_top_k, w_re,
                                r_re, shape, dtype)
    return (gw, gr) + (None,) * 8


topk_addr_forward.register_autograd(_pair_backward, setup_context=_pair_setup)


# --------------------------------------------------------------------------
# segment scan (prefill)

def _check_segment(op, addr_idx, addr_val, x, gamma, slot, mass, mask, w_top_k, r_top_k, slot_name="init_slot",
                   mass_name="init_mass") -> tuple[int, int, int, int, int]:
    """Shapes of the segment ops' arguments: (B, H, T, C, A)."""
    B, H, T, C = _dims(op, "x", x, 4)
    A = _dims(op, slot_name, slot, 4)[2]
    ev = (B, H, w_top_k + r_top_k, T)
    _check_shapes(op, addr_idx=(addr_idx, ev), addr_val=(addr_val, ev), gamma=(gamma, (B, H, T)),
                  mask=(mask, (B, T)), **{slot_name: (slot, (B, H, A, C)), mass_name: (mass, (B, H, A))})
    return B, H, T, C, A


def _segment_args(x, gamma, mask):
    x = x.contiguous()
    gamma = gamma.to(dtype=x.dtype).contiguous()
    if mask is not None:
        mask = mask.to(device=x.device, dtype=torch.bool).contiguous()
    return x, gamma, mask


def _workspace(x: Tensor, B: int, H: int, T: int, A: int, C: int, w_top_k: int, r_top_k: int) -> Tensor:
    """Per-call scan workspace (per-event records; fp32 read sums of a scan in
    slot ranges) from torch's caching allocator. A shape the scan does not
    take gets a minimal buffer: the native call then refuses it."""
    n = nat.segment_workspace_bytes(B, H, T, A, C, w_top_k, r_top_k, x.dtype) if x.dtype in nat.DTYPE_CODES else -1
    return torch.empty(max(1, n), dtype=torch.uint8, device=x.device)


@torch.library.custom_op(f"{_NS}::topk_segment_forward", mutates_args=(), device_types="cuda")
def topk_segment_forward(addr_idx: Tensor, addr_val: Tensor, x: Tensor, gamma: Tensor, init_slot: Tensor,
                         init_mass: Tensor, mask: Tensor | None, w_top_k: int, r_top_k: int, mass_aware: bool,
                         eps: float) -> tuple[Tensor, Tensor, Tensor]:
    op = "topk_segment_forward"
    _require_gpu(op, addr_idx, addr_val, x, gamma, init_slot, init_mass, mask)
    B, H, T, C, A = _check_segment(op, addr_idx, addr_val, x, gamma, init_slot, init_mass, mask, w_top_k, r_top_k)
    x, gamma, mask = _segment_args(x, gamma, mask)
    addr_idx = addr_idx.to(torch.int32).contiguous()
    addr_val = addr_val.to(torch.float32).contiguous()
    init_slot = init_slot.to(torch.float32).contiguous()
    init_mass = init_mass.to(torch.float32).contiguous()
    slot = torch.empty_like(init_slot)
    mass = torch.empty_like(init_mass)
    y = torch.empty_like(x)
    ws = _workspace(x, B, H, T, A, C, w_top_k, r_top_k)
    with torch.cuda.device(x.device):
        nat.call("ramnet_topk_segment_forward", addr_idx.data_ptr(), addr_val.data_ptr(), x.data_ptr(),
                 gamma.data_ptr(), _code(x), nat.ptr(mask), init_slot.data_ptr(), init_mass.data_ptr(),
                 slot.data_ptr(), mass.data_ptr(), y.data_ptr(), B, H, T, A, C, w_top_k, r_top_k, int(mass_aware),
                 float(eps), ws.data_ptr(), ws.numel(), nat.stream_of(x))
    return y, slot, mass


@topk_segment_forward.register_fake
def _(addr_idx, addr_val, x, gamma, init_slot, init_mass, mask, w_top_k, r_top_k, mass_aware, eps):
    return (x.new_empty(x.shape), init_slot.new_empty(init_slot.shape, dtype=torch.float32),
            init_mass.new_empty(init_mass.shape, dtype=torch.float32))


@torch.library.custom_op(f"{_NS}::topk_segment_backward", mutates_args=(), device_types="cuda")
def topk_segment_backward(addr_idx: Tensor, addr_val: Tensor, x: Tensor, gamma: Tensor, init_slot: Tensor,
                          init_mass: Tensor, mask: Tensor | None, D_y: Tensor, D_post_slot: Tensor | None,
                          D_post_mass: Tensor | None, w_top_k: int, r_top_k: int, mass_aware: bool,
                          eps: float) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Gradients of ``topk_segment_forward`` (reference op: ram_attn_ops.cpp:267-310).

    Returns (D_addr_val (B, H, Kw + Kr, T), D_x (B, H, T, C), D_gamma (B, H, T),
    D_init_slot, D_init_mass), all float32. Read rows of D_addr_val are
    gradients with respect to the positive read weights, the contract
    ``topk_addr_backward`` expects; events that do not act get 0.
    """
    _require_given("topk_segment_backward", addr_idx=addr_idx, addr_val=addr_val, x=x, gamma=gamma,
                   init_slot=init_slot, init_mass=init_mass, D_y=D_y)
    op = "topk_segment_backward"
    _require_gpu(op, addr_idx, addr_val, x, gamma, init_slot, init_mass, mask, D_y, D_post_slot, D_post_mass)
    B, H, T, C, A = _check_segment(op, addr_idx, addr_val, x, gamma, init_slot, init_mass, mask, w_top_k, r_top_k)
    _check_shapes(op, D_y=(D_y, (B, H, T, C)), D_post_slot=(D_post_slot, (B, H, A, C)),
                  D_post_mass=(D_post_mass, (B, H, A)))
    x, gamma, mask = _segment_args(x, gamma, mask)
    addr_idx = addr_idx.to(torch.int32).contiguous()
    addr_val = addr_val.to(torch.float32).contiguous()
    init_slot = init_slot.to(torch.float32).contiguous()
    init_mass = init_mass.to(torch.float32).contiguous()
    D_y = D_y.to(dtype=x.dtype).contiguous()  # as the reference, the output gradient is taken in x's dtype
    if D_post_slot is not None:
        D_post_slot = D_post_slot.to(torch.float32).contiguous()
    if D_post_mass is not None:
        D_post_mass = D_post_mass.to(torch.float32).contiguous()
    f32 = dict(dtype=torch.float32, device=x.device)
    D_addr = torch.empty((B, H, w_top_k + r_top_k, T), **f32)
    D_x = torch.empty((B, H, T, C), **f32)
    D_gamma = torch.empty((B, H, T), **f32)
    D_slot = torch.empty_like(init_slot)
    D_mass = torch.empty_like(init_mass)
    nbytes = nat.segment_backward_workspace_bytes(B, H, T, A, C, w_top_k, r_top_k)
    if nbytes < 0:
        raise RuntimeError(f"topk_segment_backward: shape not supported (A={A}, C={C}, top_k=({w_top_k}, {r_top_k}))")
    ws = torch.empty(max(1, nbytes), dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        nat.call("ramnet_topk_segment_backward", addr_idx.data_ptr(), addr_val.data_ptr(), x.data_ptr(),
                 gamma.data_ptr(), _code(x), nat.ptr(mask), init_slot.data_ptr(), init_mass.data_ptr(),
                 D_y.data_ptr(), nat.ptr(D_post_slot), nat.ptr(D_post_mass), D_addr.data_ptr(), D_x.data_ptr(),
                 D_gamma.data_ptr(), D_slot.data_ptr(), D_mass.data_ptr(), B, H, T, A, C, w_top_k, r_top_k,
                 int(mass_aware), float(eps), ws.data_ptr(), ws.numel(), nat.stream_of(x))
    return D_addr, D_x, D_gamma, D_slot, D_mass


@topk_segment_backward.register_fake
def _(addr_idx, addr_val, x, gamma, init_slot, init_mass, mask, D_y, D_post_slot, D_post_mass, w_top_k, r_top_k,
      mass_aware, eps):
    B, H, T, C = x.shape
    f32 = torch.float32
    return (x.new_empty((B, H, w_top_k + r_top_k, T), dtype=f32), x.new_empty(x.shape, dtype=f32),
            x.new_empty((B, H, T), dtype=f32), init_slot.new_empty(init_slot.shape, dtype=f32),
            init_mass.new_empty(init_mass.shape, dtype=f32))


def _segment_setup(ctx, inputs, output):
    addr_idx, addr_val, x, gamma, init_slot, init_mass, mask, w_top_k, r_top_k, mass_aware, eps = inputs
    ctx.args = (w_top_k, r_top_k, bool(mass_aware), float(eps))
    ctx.dtypes = (x.dtype, gamma.dtype, init_slot.dtype, init_mass.dtype)
    ctx.save_for_backward(addr_idx, addr_val, x, gamma, init_slot, init_mass, mask)
    ctx.set_materialize_grads(False)


def _segment_backward(ctx, D_y, D_slot, D_mass):
    """Autograd formula of ``topk_segment_forward`` (reference: _cuda_autograd.py:239-287)."""
    addr_idx, addr_val, x, gamma, init_slot, init_mass, mask = ctx.saved_tensors
    w_top_k, r_top_k, mass_aware, eps = ctx.args
    x_dt, g_dt, s_dt, m_dt = ctx.dtypes
    if D_y is None:
        D_y = torch.zeros_like(x)
    D_addr, D_x, D_gamma, D_s, D_m = topk_segment_backward(addr_idx, addr_val, x, gamma, init_slot, init_mass, mask,
                                                           D_y, D_slot, D_mass, w_top_k, r_top_k, mass_aware, eps)
    need = ctx.needs_input_grad
    return (None,
            D_addr if need[1] else None,
            D_x.to(x_dt) if need[2] else None,
            D_gamma.to(g_dt) if need[3] else None,
            D_s.to(s_dt) if need[4] else None,
            D_m.to(m_dt) if need[5] else None) + (None,) * 5


topk_segment_forward.register_autograd(_segment_backward, setup_context=_segment_setup)


# --------------------------------------------------------------------------
# training pair with saved rows (no reference counterpart: the reference's
# backward reconstructs the forward). Same results as topk_segment_forward /
# topk_segment_backward; the forward also keeps, per event, the row its
# backward would otherwise recompute.

def _saved_bytes(op: str, B: int, H: int, T: int, A: int, C: int, w_top_k: int, r_top_k: int,
                 dtype: torch.dtype) -> int:
    n = nat.segment_saved_bytes(B, H, T, A, C, w_top_k, r_top_k, dtype)
    if n < 0:
        raise RuntimeError(f"{op}: no saved-row form for this shape (A={A}, C={C}, top_k=({w_top_k}, {r_top_k})); "
                           "use topk_segment_forward")
    return n


@torch.library.custom_op(f"{_NS}::topk_segment_forward_saved", mutates_args=(), device_types="cuda")
def topk_segment_forward_saved(addr_idx: Tensor, addr_val: Tensor, x: Tensor, gamma: Tensor, init_slot: Tensor,
                               init_mass: Tensor, mask: Tensor | None, w_top_k: int, r_top_k: int, mass_aware: bool,
                               eps: float) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """``topk_segment_forward`` that also returns ``saved`` (uint8): the scan
    records and, per event, x - s before each write and the row of each
    read, which ``topk_segment_backward_saved`` takes instead of replaying
    the forward. Raises RuntimeError where
    ``ramnet_ops._native.segment_saved_bytes`` is -1."""
    op = "topk_segment_forward_saved"
    _require_gpu(op, addr_idx, addr_val, x, gamma, init_slot, init_mass, mask)
    B, H, T, C, A = _check_segment(op, addr_idx, addr_val, x, gamma, init_slot, init_mass, mask, w_top_k, r_top_k)
    x, gamma, mask = _segment_args(x, gamma, mask)
    nbytes = _saved_bytes(op, B, H, T, A, C, w_top_k, r_top_k, x.dtype)
    addr_idx = addr_idx.to(torch.int32).contiguous()
    addr_val = addr_val.to(torch.float32).contiguous()
    init_slot = init_slot.to(torch.float32).contiguous()
    init_mass = init_mass.to(torch.float32).contiguous()
    slot = torch.empty_like(init_slot)
    mass = torch.empty_like(init_mass)
    y = torch.empty_like(x)
    ws = _workspace(x, B, H, T, A, C, w_top_k, r_top_k)
    saved = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        nat.call("ramnet_topk_segment_forward_save", addr_idx.data_ptr(), addr_val.data_ptr(), x.data_ptr(),
                 gamma.data_ptr(), _code(x), nat.ptr(mask), init_slot.data_ptr(), init_mass.data_ptr(),
                 slot.data_ptr(), mass.data_ptr(), y.data_ptr(), B, H, T, A, C, w_top_k, r_top_k, int(mass_aware),
                 float(eps), ws.data_ptr(), ws.numel(), saved.data_ptr(), saved.numel(), nat.stream_of(x))
    return y, slot, mass, saved


@topk_segment_forward_saved.register_fake
def _(addr_idx, addr_val, x, gamma, init_slot, init_mass, mask, w_top_k, r_top_k, mass_aware, eps):
    B, H, T, C = x.shape
    A = init_slot.shape[2]
    nbytes = _saved_bytes("topk_segment_forward_saved", B, H, T, A, C, w_top_k, r_top_k, x.dtype)
    return (x.new_empty(x.shape), init_slot.new_empty(init_slot.shape, dtype=torch.float32),
            init_mass.new_empty(init_mass.shape, dtype=torch.float32), x.new_empty((nbytes,), dtype=torch.uint8))


@torch.library.custom_op(f"{_NS}::topk_segment_backward_saved", mutates_args=(), device_types="cuda")
def topk_segment_backward_saved(addr_val: Tensor, x: Tensor, gamma: Tensor, init_slot: Tensor, init_mass: Tensor,
                                saved: Tensor, D_y: Tensor, D_post_slot: Tensor | None, D_post_mass: Tensor | None,
                                w_top_k: int, r_top_k: int, mass_aware: bool,
                                eps: float) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Gradients of ``topk_segment_forward_saved`` from its ``saved`` rows;
    outputs as ``topk_segment_backward``."""
    op = "topk_segment_backward_saved"
    _require_given(op, addr_val=addr_val, x=x, gamma=gamma, init_slot=init_slot, init_mass=init_mass, saved=saved,
                   D_y=D_y)
    _require_gpu(op, addr_val, x, gamma, init_slot, init_mass, saved, D_y, D_post_slot, D_post_mass)
    B, H, T, C = _dims(op, "x", x, 4)
    A = _dims(op, "init_slot", init_slot, 4)[2]
    K = w_top_k + r_top_k
    _check_shapes(op, addr_val=(addr_val, (B, H, K, T)), gamma=(gamma, (B, H, T)), init_slot=(init_slot, (B, H, A, C)),
                  init_mass=(init_mass, (B, H, A)), D_y=(D_y, (B, H, T, C)), D_post_slot=(D_post_slot, (B, H, A, C)),
                  D_post_mass=(D_post_mass, (B, H, A)))
    x, gamma, _ = _segment_args(x, gamma, None)
    nbytes = _saved_bytes(op, B, H, T, A, C, w_top_k, r_top_k, x.dtype)
    if saved.dtype != torch.uint8 or saved.numel() < nbytes or not saved.is_contiguous():
        raise RuntimeError(f"{op}: saved must be the contiguous uint8 tensor of topk_segment_forward_saved")
    addr_val = addr_val.to(torch.float32).contiguous()
    init_slot = init_slot.to(torch.float32).contiguous()
    init_mass = init_mass.to(torch.float32).contiguous()
    D_y = D_y.to(dtype=x.dtype).contiguous()
    if D_post_slot is not None:
        D_post_slot = D_post_slot.to(torch.float32).contiguous()
    if D_post_mass is not None:
        D_post_mass = D_post_mass.to(torch.float32).contiguous()
    f32 = dict(dtype=torch.float32, device=x.device)
    D_addr = torch.empty((B, H, K, T), **f32)
    D_x = torch.empty((B, H, T, C), **f32)
    D_gamma = torch.empty((B, H, T), **f32)
    D_slot = torch.empty_like(init_slot)
    D_mass = torch.empty_like(init_mass)
    ws = torch.empty(max(1, nat.segment_backward_saved_workspace_bytes(B, H, T, A, C, w_top_k, r_top_k)),
                     dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        nat.call("ramnet_topk_segment_backward_saved", addr_val.data_ptr(), x.data_ptr(), gamma.data_ptr(), _code(x),
                 init_slot.data_ptr(), init_mass.data_ptr(), D_y.data_ptr(), nat.ptr(D_post_slot),
                 nat.ptr(D_post_mass), D_addr.data_ptr(), D_x.data_ptr(), D_gamma.data_ptr(), D_slot.data_ptr(),
                 D_mass.data_ptr(), B, H, T, A, C, w_top_k, r_top_k, int(mass_aware), float(eps), saved.data_ptr(),
                 saved.numel(), ws.data_ptr(), ws.numel(), nat.stream_of(x))
    return D_addr, D_x, D_gamma, D_slot, D_mass


@topk_segment_backward_saved.register_fake
def _(addr_val, x, gamma, init_slot, init_mass, saved, D_y, D_post_slot, D_post_mass, w_top_k, r_top_k, mass_aware,
      eps):
    B, H, T, C = x.shape
    f32 = torch.float32
    return (x.new_empty((B, H, w_top_k + r_top_k, T), dtype=f32), x.new_empty(x.shape, dtype=f32),
            x.new_empty((B, H, T), dtype=f32), init_slot.new_empty(init_slot.shape, dtype=f32),
            init_mass.new_empty(init_mass.shape, dtype=f32))


def _segment_saved_setup(ctx, inputs, output):
    addr_idx, addr_val, x, gamma, init_slot, init_mass, mask, w_top_k, r_top_k, mass_aware, eps = inputs
    ctx.args = (w_top_k, r_top_k, bool(mass_aware), float(eps))
    ctx.dtypes = (x.dtype, gamma.dtype, init_slot.dtype, init_mass.dtype)
    ctx.save_for_backward(addr_val, x, gamma, init_slot, init_mass, output[3])  # saved: uint8, no gradient
    ctx.set_materialize_grads(False)


def _segment_saved_backward(ctx, D_y, D_slot, D_mass, D_saved):
    addr_val, x, gamma, init_slot, init_mass, saved = ctx.saved_tensors
    w_top_k, r_top_k, mass_aware, eps = ctx.args
    x_dt, g_dt, s_dt, m_dt = ctx.dtypes
    if D_y is None:
        D_y = torch.zeros_like(x)
    D_addr, D_x, D_gamma, D_s, D_m = topk_segment_backward_saved(addr_val, x, gamma, init_slot, init_mass, saved, D_y,
                                                                 D_slot, D_mass, w_top_k, r_top_k, mass_aware, eps)
    need = ctx.needs_input_grad
    return (None,
            D_addr if need[1] else None,
            D_x.to(x_dt) if need[2] else None,
            D_gamma.to(g_dt) if need[3] else None,
            D_s.to(s_dt) if need[4] else None,
            D_m.to(m_dt) if need[5] else None) + (None,) * 5


topk_segment_forward_saved.register_autograd(_segment_saved_backward, setup_context=_segment_saved_setup)


@torch.library.custom_op(f"{_NS}::topk_segment_forward_", mutates_args=("slot", "mass"), device_types="cuda")
def topk_segment_forward_(addr_idx: Tensor, addr_val: Tensor, x: Tensor, gamma: Tensor, slot: Tensor, mass: Tensor,
                          mask: Tensor | None, w_top_k: int, r_top_k: int, mass_aware: bool, eps: float) -> Tensor:
    op = "topk_segment_forward_"
    _require_gpu(op, addr_idx, addr_val, x, gamma, slot, mass, mask)
    B, H, T, C, A = _check_segment(op, addr_idx, addr_val, x, gamma, slot, mass, mask, w_top_k, r_top_k, "slot",
                                   "mass")
    _require_state(op, slot, mass)
    x, gamma, mask = _segment_args(x, gamma, mask)
    addr_idx = addr_idx.to(torch.int32).contiguous()
    addr_val = addr_val.to(torch.float32).contiguous()
    # channel slices of one head may start after another has stored the new
    # masses, so every slice reads the masses from a snapshot
    mass_in = mass.clone()
    y = torch.empty_like(x)
    ws = _workspace(x, B, H, T, A, C, w_top_k, r_top_k)
    with torch.cuda.device(x.device):
        nat.call("ramnet_topk_segment_forward_", addr_idx.data_ptr(), addr_val.data_ptr(), x.data_ptr(),
                 gamma.data_ptr(), _code(x), nat.ptr(mask), slot.data_ptr(), mass.data_ptr(), mass_in.data_ptr(),
                 y.data_ptr(), B, H, T, A, C, w_top_k, r_top_k, int(mass_aware), float(eps), ws.data_ptr(),
                 ws.numel(), nat.stream_of(x))
    return y


@topk_segment_forward_.register_fake
def _(addr_idx, addr_val, x, gamma, slot, mass, mask, w_top_k, r_top_k, mass_aware, eps):
    return x.new_empty(x.shape)


def _require_state(name: str, slot: Tensor, mass: Tensor) -> None:
    if slot.dtype != torch.float32 or mass.dtype != torch.float32 or not (slot.is_contiguous() and mass.is_contiguous()):
        raise RuntimeError(f"{name}: slot and mass must be contiguous float32 tensors")


def _check_ram_attn(op, w_addr, r_addr, x, gamma, slot, mass, mask, position_ids, slot_name="init_slot",
                    mass_name="init_mass") -> None:
    B, H, U, P, T = _dims(op, "w_addr", w_addr, 5)
    C = _dims(op, "x", x, 4)[-1]
    A = P ** U
    _check_shapes(op, r_addr=(r_addr, (B, H, U, P, T)), x=(x, (B, H, T, C)), gamma=(gamma, (B, H, T)),
                  mask=(mask, (B, T)), position_ids=(position_ids, (B, T)),
                  **{slot_name: (slot, (B, H, A, C)), mass_name: (mass, (B, H, A))})


def _ram_attn_call(w_addr, r_addr, x, gamma, mask, embed_num, position_ids, init_slot, init_mass, slot, mass,
                   w_top_k, r_top_k, w_re_norm, r_re_norm, mass_aware, eps):
    B, H, U, P, T = w_addr.shape
    C = x.shape[-1]
    A = P ** U
    if r_addr.dtype != w_addr.dtype or x.dtype != w_addr.dtype:
        raise RuntimeError("ram_attn_forward: w_addr, r_addr and x must share dtype and address shape")
    w_addr, r_addr = w_addr.contiguous(), r_addr.contiguous()
    x, gamma, mask = _segment_args(x, gamma, mask)
    pos = position_ids.to(device=x.device, dtype=torch.int32).contiguous()
    y = torch.empty_like(x)
    ws = _workspace(x, B, H, T, A, C, w_top_k, r_top_k)
    with torch.cuda.device(x.device):
        nat.call("ramnet_ram_attn_forward", w_addr.data_ptr(), r_addr.data_ptr(), x.data_ptr(), gamma.data_ptr(),
                 _code(x), nat.ptr(mask), embed_num, pos.data_ptr(), init_slot.data_ptr(), init_mass.data_ptr(),
                 slot.data_ptr(), mass.data_ptr(), y.data_ptr(), B, H, U, P, T, A, C, w_top_k, r_top_k,
                 float(w_re_norm), float(r_re_norm), int(mass_aware), float(eps), ws.data_ptr(), ws.numel(),
                 nat.stream_of(x))
    return y


@torch.library.custom_op(f"{_NS}::ram_attn_forward", mutates_args=(), device_types="cuda")
def ram_attn_forward(w_addr: Tensor, r_addr: Tensor, x: Tensor, gamma: Tensor, init_slot: Tensor, init_mass: Tensor,
                     mask: Tensor | None, embed_num: int, position_ids: Tensor, w_top_k: int, r_top_k: int,
                     w_re_norm: float, r_re_norm: float, mass_aware: bool,
                     eps: float) -> tuple[Tensor, Tensor, Tensor]:
    """Whole parallel forward (decoders + segment scan) returning y, new slot and mass."""
    _require_gpu("ram_attn_forward", w_addr, r_addr, x, gamma, init_slot, init_mass, position_ids, mask)
    _check_ram_attn("ram_attn_forward", w_addr, r_addr, x, gamma, init_slot, init_mass, mask, position_ids)
    init_slot = init_slot.to(torch.float32).contiguous()
    init_mass = init_mass.to(torch.float32).contiguous()
    slot = torch.empty_like(init_slot)
    mass = torch.empty_like(init_mass)
    y = _ram_attn_call(w_addr, r_addr, x, gamma, mask, embed_num, position_ids, init_slot, init_mass, slot, mass,
                       w_top_k, r_top_k, w_re_norm, r_re_norm, mass_aware, eps)
    return y, slot, mass


@ram_attn_forward.register_fake
def _(w_addr, r_addr, x, gamma, init_slot, init_mass, mask, embed_num, position_ids, w_top_k, r_top_k, w_re_norm,
      r_re_norm, mass_aware, eps):
    return (x.new_empty(x.shape), init_slot.new_empty(init_slot.shape, dtype=torch.float32),
            init_mass.new_empty(init_mass.shape, dtype=torch.float32))


@torch.library.custom_op(f"{_NS}::ram_attn_forward_", mutates_args=("slot", "mass"), device_types="cuda")
def ram_attn_forward_(w_addr: Tensor, r_addr: Tensor, x: Tensor, gamma: Tensor, slot: Tensor, mass: Tensor,
                      mask: Tensor | None, embed_num: int, position_ids: Tensor, w_top_k: int, r_top_k: int,
                      w_re_norm: float, r_re_norm: float, mass_aware: bool, eps: float) -> Tensor:
    """In-place whole parallel forward: updates slot and mass, returns y."""
    _require_gpu("ram_attn_forward_", w_addr, r_addr, x, gamma, slot, mass, position_ids, mask)
    _check_ram_attn("ram_attn_forward_", w_addr, r_addr, x, gamma, slot, mass, mask, position_ids, "slot", "mass")
    _require_state("ram_attn_forward_", slot, mass)
    mass_in = mass.clone()  # see topk_segment_forward_
    return _ram_attn_call(w_addr, r_addr, x, gamma, mask, embed_num, position_ids, slot, mass_in, slot, mass,
                          w_top_k, r_top_k, w_re_norm, r_re_norm, mass_aware, eps)


@ram_attn_forward_.register_fake
def _(w_addr, r_addr, x, gamma, slot, mass, mask, embed_num, position_ids, w_top_k, r_top_k, w_re_norm, r_re_norm,
      mass_aware, eps):
    return x.new_empty(x.shape)


# --------------------------------------------------------------------------
# fused decode step

@torch.library.custom_op(f"{_NS}::topk_autoregressive_", mutates_args=("slot", "mass"), device_types="cuda")
def topk_autoregressive_(w_addr: Tensor, r_addr: Tensor, x: Tensor, gamma: Tensor, slot: Tensor, mass: Tensor,
                         mask: Tensor, embed_num: int, position_ids: Tensor, w_top_k: int, r_top_k: int,
                         w_re_norm: float, r_re_norm: float, mass_aware: bool, eps: float) -> Tensor:
    op = "topk_autoregressive_"
    _require_gpu(op, w_addr, r_addr, x, gamma, slot, mass, position_ids)
    B, H, U, P = _dims(op, "w_addr", w_addr, 4)
    C = _dims(op, "x", x, 3)[-1]
    A = _dims(op, "slot", slot, 4)[2]
    _check_slots(op, U, P, A)
    _check_shapes(op, r_addr=(r_addr, (B, H, U, P)), x=(x, (B, H, C)), gamma=(gamma, (B, H)),
                  slot=(slot, (B, H, A, C)), mass=(mass, (B, H, A)), position_ids=(position_ids, (B,)),
                  mask=(None if mask is None or mask.numel() == 0 else mask, (B,)))
    _require_state(op, slot, mass)
    _check_decode_dtypes(op, w_addr, r_addr, x)
    w_addr, r_addr, x = w_addr.contiguous(), r_addr.contiguous(), x.contiguous()
    gamma = gamma.to(dtype=x.dtype).contiguous()
    pos = position_ids.to(device=x.device, dtype=torch.int32).contiguous()
    m = None if mask is None or mask.numel() == 0 else mask.to(device=x.device, dtype=torch.bool).contiguous()
    y = torch.empty_like(x)
    with torch.cuda.device(x.device):
        nat.call("ramnet_topk_autoregressive_", w_addr.data_ptr(), r_addr.data_ptr(), x.data_ptr(), gamma.data_ptr(),
                 _code(x), slot.data_ptr(), mass.data_ptr(), nat.ptr(m), embed_num, pos.data_ptr(), B, H, U, P, A, C,
                 w_top_k, r_top_k, float(w_re_norm), float(r_re_norm), int(mass_aware), float(eps), y.data_ptr(),
                 nat.stream_of(x))
    return y


@topk_autoregressive_.register_fake
def _(w_addr, r_addr, x, gamma, slot, mass, mask, embed_num, position_ids, w_top_k, r_top_k, w_re_norm, r_re_norm,
      mass_aware, eps):
    return x.new_empty(x.shape)


@torch.library.custom_op(f"{_NS}::topk_autoregressive_steps_", mutates_args=("slot", "mass"), device_types="cuda")
def topk_autoregressive_steps_(w_addr: Tensor, r_addr: Tensor, x: Tensor, gamma: Tensor, slot: Tensor, mass: Tensor,
                               mask: Tensor, embed_num: int, position_ids: Tensor, w_top_k: int, r_top_k: int,
                               w_re_norm: float, r_re_norm: float, mass_aware: bool, eps: float) -> Tensor:
    """S consecutive ``topk_autoregressive_`` steps in one call: every input
    carries a leading step dimension (w_addr/r_addr (S, B, H, U, P), x
    (S, B, H, C), gamma (S, B, H), position_ids and mask (S, B)) and y is
    (S, B, H, C). This library's multi-step form of the reference decode op
    (ram_attn_ops.cpp:349-394), which has no such variant: the kernel walks
    the steps of each (b, h) in one launch."""
    op = "topk_autoregressive_steps_"
    _require_gpu(op, w_addr, r_addr, x, gamma, slot, mass, position_ids)
    S, B, H, U, P = _dims(op, "w_addr", w_addr, 5)
    C = _dims(op, "x", x, 4)[-1]
    A = _dims(op, "slot", slot, 4)[2]
    _check_slots(op, U, P, A)
    _check_shapes(op, r_addr=(r_addr, (S, B, H, U, P)), x=(x, (S, B, H, C)), gamma=(gamma, (S, B, H)),
                  slot=(slot, (B, H, A, C)), mass=(mass, (B, H, A)), position_ids=(position_ids, (S, B)),
                  mask=(None if mask is None or mask.numel() == 0 else mask, (S, B)))
    _require_state(op, slot, mass)
    _check_decode_dtypes(op, w_addr, r_addr, x)
    w_addr, r_addr, x = w_addr.contiguous(), r_addr.contiguous(), x.contiguous()
    gamma = gamma.to(dtype=x.dtype).contiguous()
    pos = position_ids.to(device=x.device, dtype=torch.int32).contiguous()
    m = None if mask is None or mask.numel() == 0 else mask.to(device=x.device, dtype=torch.bool).contiguous()
    y = torch.empty_like(x)
    with torch.cuda.device(x.device):
        nat.call("ramnet_topk_autoregressive_steps_", w_addr.data_ptr(), r_addr.data_ptr(), x.data_ptr(),
                 gamma.data_ptr(), _code(x), slot.data_ptr(), mass.data_ptr(), nat.ptr(m), embed_num, pos.data_ptr(),
                 S, B, H, U, P, A, C, w_top_k, r_top_k, float(w_re_norm), float(r_re_norm), int(mass_aware),
                 float(eps), y.data_ptr(), nat.stream_of(x))
    return y


@topk_autoregressive_steps_.register_fake
def _(w_addr, r_addr, x, gamma, slot, mass, mask, embed_num, position_ids, w_top_k, r_top_k, w_re_norm, r_re_norm,
      mass_aware, eps):
    return x.new_empty(x.shape)

"""GPU backend of ``ramnet_ops`` on MI355X: dispatch to the gfx950 operators.

Mirrors the reference's op glue (packages/ramnet-ops/src/ramnet_ops/impl/
cuda_impl.py:11-333): the same entry points, argument checks and error
types, and the same path choice -- a single token without gradients runs the
fused decode step, everything else runs the address decoder followed by the
time-ordered segment scan. Differences by design:

* no padding of T to a multiple of 32 (the HIP kernels take any T);
* no event grouping (``gather_segment``'s global sort): the segment scan walks
  tokens in order with the slot state resident in LDS;
* with inputs that require grad (and grad mode on) the forward runs the two
  autograd-registered ops ``topk_addr_forward`` and ``topk_segment_forward``,
  as the reference does, so their backward kernels
  (``topk_addr_backward``, ``topk_segment_backward``) give the gradients;
  without gradients it runs the fused decoder + scan op.
"""
from __future__ import annotations

import torch

from .. import _native as nat
from . import _ops
from ._cuda_config import ADDRESS_LIMIT, check_int_capacity

ops = _ops  # the registered torch.ops.ramnet_ops.* operators


def _cuda_topk_autoregressive_(
        w_addr: torch.Tensor,  # (B, H, U, P)
        r_addr: torch.Tensor,  # (B, H, U, P)
        x: torch.Tensor,  # (B, H, C)
        gamma: torch.Tensor,  # (B, H)
        slot_: torch.Tensor,  # r/w (B, H, A, C) fp32
        mass_: torch.Tensor,  # r/w (B, H, A) fp32
        mask: torch.Tensor | None,  # (B)
        embed_num: int,
        position_ids: torch.Tensor,  # (B)
        w_top_k: int,
        r_top_k: int,
        w_re_norm: float,
        r_re_norm: float,
        mass_aware: bool,
        eps: float,
) -> torch.Tensor:  # (B, H, C)
    """One fused decode step; updates ``slot_`` and ``mass_`` in place."""
    assert slot_.is_contiguous() and mass_.is_contiguous(), \
        f"Expected contiguous state, got slot={slot_.is_contiguous()}, mass={mass_.is_contiguous()}."
    empty = torch.empty(0, dtype=torch.bool, device=x.device)
    mask = empty if mask is None else mask.to(device=x.device, dtype=torch.bool).contiguous()
    return torch.ops.ramnet_ops.topk_autoregressive_(
        w_addr.contiguous(), r_addr.contiguous(), x.contiguous(), gamma.contiguous(), slot_, mass_,
        mask, embed_num, position_ids.contiguous(), w_top_k, r_top_k, w_re_norm, r_re_norm, mass_aware, eps)


def _cuda_ram_attn(
        w_addr: torch.Tensor,  # (B, H, U, P, T)
        r_addr: torch.Tensor,  # (B, H, U, P, T)
        xs: torch.Tensor,  # (B, H, T, C)
        gamma: torch.Tensor,  # (B, H, T)
        init_slot: torch.Tensor,  # (B, H, A, C)
        init_mass: torch.Tensor,  # (B, H, A)
        mask: torch.Tensor | None,  # (B, T)
        embed_num: int,
        position_ids: torch.Tensor,  # (B, T)
        top_k: tuple[int, int] | None,
        top_k_re_norm: tuple[float, float],
        mass_aware: bool,
        eps: float,
        inplace: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:  # (B, H, T, C), (B, H, A, C), (B, H, A)
    """RAM attention on the HIP operators (reference: cuda_impl.py:144-276)."""
    assert xs.ndim == 4 and w_addr.ndim == 5 and r_addr.ndim == 5, \
        f"Expected xs (B, H, T, C), w/r (B, H, U, P, T); got {tuple(xs.shape)}, {tuple(w_addr.shape)}, {tuple(r_addr.shape)}."
    if top_k is None:
        raise ValueError("CUDA RAM attention only supports Top-K mode; dense mode (top_k=None) is not implemented on MI355X.")
    assert isinstance(top_k, tuple) and len(top_k) == 2 and all(isinstance(k, int) and k > 0 for k in top_k), \
        f"Expected top_k=(positive write_k, positive read_k), got {top_k!r}."
    assert isinstance(top_k_re_norm, tuple) and len(top_k_re_norm) == 2 \
        and all(isinstance(v, (int, float)) and 0 <= v <= 1 for v in top_k_re_norm), \
        f"Expected top_k_re_norm=(w, r) in [0, 1], got {top_k_re_norm!r}."

    B, H, T, C = xs.shape
    U, P = w_addr.shape[2], w_addr.shape[3]
    A = P ** U
    w_top_k, r_top_k = top_k
    w_re, r_re = (float(v) for v in top_k_re_norm)
    assert all(k <= A for k in top_k), f"Expected top_k <= A={A}, got {top_k}."
    assert isinstance(embed_num, int) and 0 <= embed_num <= H, f"Expected embed_num in [0, {H}], got {embed_num!r}."
    assert A < ADDRESS_LIMIT, f"Address space overflow: A={A}, limit={ADDRESS_LIMIT}."
    check_int_capacity(B, H, U, P, A, C, T, embed_num, w_top_k, r_top_k,
                       B * H * U * P * T, B * H * A * C, B * H * T * C, B * H * T * (w_top_k + r_top_k))

    requires_grad = torch.is_grad_enabled() and any(
        t.requires_grad for t in (w_addr, r_addr, xs, gamma, init_slot, init_mass))
    position_ids = position_ids.to(device=xs.device, dtype=torch.int32)
    if mask is not None:
        mask = mask.to(device=xs.device, dtype=torch.bool)

    assert w_addr.dtype == r_addr.dtype == xs.dtype == gamma.dtype, \
        f"Expected matching dtypes, got w={w_addr.dtype}, r={r_addr.dtype}, x={xs.dtype}, gamma={gamma.dtype}."
    assert w_addr.device == r_addr.device == xs.device == gamma.device == init_slot.device == init_mass.device \
        == position_ids.device, "Expected all inputs on one device."
    expected_shapes = (
        ("w_addr", w_addr, (B, H, U, P, T)),
        ("r_addr", r_addr, (B, H, U, P, T)),
        ("xs", xs, (B, H, T, C)),
        ("gamma", gamma, (B, H, T)),
        ("position_ids", position_ids, (B, T)),
        ("init_slot", init_slot, (B, H, A, C)),
        ("init_mass", init_mass, (B, H, A)),
    )
    for name, tensor, shape in expected_shapes:
        assert tuple(tensor.shape) == shape, f"Expected {name}.shape == {shape}, but got {tuple(tensor.shape)}."
    assert mask is None or tuple(mask.shape) == (B, T), f"Expected mask.shape={(B, T)}, got {tuple(mask.shape)}."

    acc_type = torch.float32 if xs.dtype in (torch.float16, torch.bfloat16) else xs.dtype
    if acc_type != torch.float32:
        raise RuntimeError(f"ramnet_ops on MI355X supports float32, float16 and bfloat16 inputs, got {xs.dtype}.")
    if inplace:
        assert not requires_grad, "inplace=True does not support backward."
        assert init_slot.dtype == init_mass.dtype == acc_type, \
            f"Expected inplace state dtype={acc_type}, got slot={init_slot.dtype}, mass={init_mass.dtype}."
        assert init_slot.is_contiguous() and init_mass.is_contiguous(), "Expected contiguous inplace state."

    if requires_grad:
        # the differentiable composition (reference: cuda_impl.py:252-271).
        # Where the shape allows it, the segment forward keeps the rows its
        # backward needs (topk_segment_forward_saved), so the backward runs
        # one pass over the sequence instead of replaying the forward first.
        # Graphs traced by torch.compile keep the reference-shaped ops: the
        # size query is a native call the tracer does not follow.
        addr_idx, addr_val = torch.ops.ramnet_ops.topk_addr_forward(
            w_addr, r_addr, embed_num, A, position_ids, w_top_k, r_top_k, w_re, r_re)
        if not torch.compiler.is_compiling() and \
                nat.segment_saved_bytes(B, H, T, A, C, w_top_k, r_top_k, xs.dtype) >= 0:
            ys, post_slot, post_mass, _ = torch.ops.ramnet_ops.topk_segment_forward_saved(
                addr_idx, addr_val, xs, gamma, init_slot, init_mass, mask, w_top_k, r_top_k, mass_aware, eps)
            return ys, post_slot, post_mass
        return torch.ops.ramnet_ops.topk_segment_forward(
            addr_idx, addr_val, xs, gamma, init_slot, init_mass, mask, w_top_k, r_top_k, mass_aware, eps)

    if T == 1:
        with torch.no_grad():
            post_slot = init_slot if inplace else init_slot.to(dtype=acc_type, memory_format=torch.contiguous_format, copy=True)
            post_mass = init_mass if inplace else init_mass.to(dtype=acc_type, memory_format=torch.contiguous_format, copy=True)
            ys = _cuda_topk_autoregressive_(
                w_addr.squeeze(-1), r_addr.squeeze(-1), xs.squeeze(-2), gamma.squeeze(-1), post_slot, post_mass,
                None if mask is None else mask.squeeze(-1), embed_num, position_ids.squeeze(-1),
                w_top_k, r_top_k, w_re, r_re, mass_aware, eps)
        return ys.unsqueeze(-2), post_slot, post_mass

    # decoders + segment scan in one native call; the decoders hand the scan
    # its per-event records directly
    if inplace:
        ys = torch.ops.ramnet_ops.ram_attn_forward_(
            w_addr, r_addr, xs, gamma, init_slot, init_mass, mask, embed_num, position_ids, w_top_k, r_top_k,
            w_re, r_re, mass_aware, eps)
        return ys, init_slot, init_mass
    ys, post_slot, post_mass = torch.ops.ramnet_ops.ram_attn_forward(
        w_addr, r_addr, xs, gamma, init_slot, init_mass, mask, embed_num, position_ids, w_top_k, r_top_k,
        w_re, r_re, mass_aware, eps)
    return ys, post_slot, post_mass


def _cuda_topk_addr(
        addr: torch.Tensor,  # (B, H, U, P, T)
        embed_num: int,
        position_ids: torch.Tensor,  # (B, T)
        top_k: int,
        top_k_re_norm: float,
        addr_val_neg: bool = False,
        encode_batch_idx: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:  # int32 (B, H, K, T), float32 (B, H, K, T)
    """Decode one address tensor (reference: cuda_impl.py:279-333).

    Indices encode ``(b * H + h) * A + a`` by default, ``h * A + a`` with
    ``encode_batch_idx=False``; CAPE offsets apply in both modes.
    """
    assert addr.ndim == 5, f"Expected address shape (B, H, U, P, T), got {tuple(addr.shape)}."
    assert addr.is_cuda, f"Expected GPU addresses, got {addr.device}."
    B, H, U, P, T = addr.shape
    A = P ** U
    assert A < ADDRESS_LIMIT, f"Address space overflow: A={A}, limit={ADDRESS_LIMIT}."
    assert isinstance(top_k, int) and 0 < top_k <= A, f"Expected top_k in [1, A={A}], got {top_k!r}."
    assert isinstance(embed_num, int) and 0 <= embed_num <= H, f"Expected embed_num in [0, {H}], got {embed_num!r}."
    assert isinstance(top_k_re_norm, (int, float)) and 0 <= top_k_re_norm <= 1, \
        f"Expected top_k_re_norm in [0, 1], got {top_k_re_norm!r}."
    assert isinstance(addr_val_neg, bool), f"Expected boolean addr_val_neg, got {addr_val_neg!r}."
    assert isinstance(encode_batch_idx, bool), f"Expected boolean encode_batch_idx, got {encode_batch_idx!r}."
    assert tuple(position_ids.shape) == (B, T), f"Expected position_ids.shape={(B, T)}, got {tuple(position_ids.shape)}."
    check_int_capacity(B, H, U, P, A, T, embed_num, top_k, B * H * U * P * T, B * H * A, B * H * top_k * T)
    position_ids = position_ids.to(device=addr.device, dtype=torch.int32)
    return torch.ops.ramnet_ops.topk_addr_single_forward(
        addr, embed_num, A, position_ids, top_k, float(top_k_re_norm), addr_val_neg, encode_batch_idx)

"""Public RAM-Net operator API: ``random_access_memory_attention`` and ``topk_addr``.

Signatures, argument validation, default filling, broadcasting and error
types follow the reference API (packages/ramnet-ops/src/ramnet_ops/
ram_attn.py:46-367) so callers such as ``RAMNetAttention.forward_with_state``
(ram_attn_block.py:332-340) run unchanged. The compute backend is the gfx950
HIP operator library; PyTorch-ROCm reports HIP devices as ``cuda``, so
``impl_backend='cuda'`` selects it.

This package ships no CPU implementation. Inputs that the HIP backend cannot
take (CPU tensors, dense ``top_k=None`` mode, ``impl_backend='torch'``) raise
an error instead of falling back.
"""
from __future__ import annotations

from typing import Literal

import torch

try:
    from .impl.cuda_impl import _cuda_ram_attn, _cuda_topk_addr
    _load_error: Exception | None = None
except ImportError as exc:  # library not built: fail at call time with the cause attached
    _cuda_ram_attn = None
    _cuda_topk_addr = None
    _load_error = exc

_HIP_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def get_broadcast(*vals: int) -> int:
    """The one non-singleton size among broadcast-compatible dimensions (1 if none)."""
    sizes = set(vals) - {1}
    assert len(sizes) <= 1, f"Cannot broadcast {vals}"
    return sizes.pop() if sizes else 1


def _unavailable(what: str) -> RuntimeError:
    err = RuntimeError(f"{what}: the MI355X HIP operator library could not be loaded.")
    err.__cause__ = _load_error
    return err


def _no_torch_backend(what: str) -> RuntimeError:
    return RuntimeError(
        f"{what}: impl_backend='torch' (the dense pure-PyTorch reference) is not part of this package; "
        "use impl_backend='cuda' or None with GPU tensors.")


def topk_addr(
        addr: torch.Tensor,
        embed_num: int,
        position_ids: torch.Tensor,
        top_k: int,
        top_k_re_norm: float,
        addr_val_neg: bool = False,
        encode_batch_idx: bool = True,
        impl_backend: Literal['torch', 'cuda'] | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-K address decoding.

    :param addr: Address logits in (B, H, U, P, T); A = P ** U slots.
    :param embed_num: Heads ``h < embed_num`` use the CAPE cyclic shift.
    :param position_ids: (B, T) token positions for CAPE.
    :param top_k: Number of addresses kept, in ``[1, A]``.
    :param top_k_re_norm: r in [0, 1]; kept probabilities q become q / sum(q) ** r.
    :param addr_val_neg: Negate the returned weights.
    :param encode_batch_idx: Indices ``(b * H + h) * A + a``; False gives ``h * A + a``.
    :param impl_backend: 'cuda' (HIP) or None.
    :return: ``(idx int32, val float32)``, both (B, H, K, T).
    """
    assert isinstance(addr, torch.Tensor), f"Expected addr to be Tensor, got {type(addr).__name__}."
    if not isinstance(top_k_re_norm, (int, float)):
        raise TypeError("`top_k_re_norm` must be a number in [0, 1].")
    if not 0 <= top_k_re_norm <= 1:
        raise ValueError("`top_k_re_norm` must be in [0, 1].")
    if impl_backend not in (None, 'torch', 'cuda'):
        raise ValueError(f"Unsupported impl_backend: {impl_backend!r}.")
    if impl_backend == 'torch':
        raise _no_torch_backend("topk_addr")
    if _cuda_topk_addr is None:
        raise _unavailable("topk_addr")
    if not addr.is_cuda or addr.dtype not in _HIP_DTYPES:
        raise RuntimeError(f"topk_addr needs a float16/bfloat16/float32 GPU tensor, got {addr.dtype} on {addr.device}.")
    return _cuda_topk_addr(addr, embed_num, position_ids, top_k, float(top_k_re_norm), addr_val_neg, encode_batch_idx)


def _as_pair(value, kind, message: str) -> tuple:
    if isinstance(value, kind):
        return value, value
    if isinstance(value, (tuple, list)) and len(value) == 2 and all(isinstance(v, kind) for v in value):
        return tuple(value)
    raise TypeError(message)


def random_access_memory_attention(
        w_addr: torch.Tensor,
        r_addr: torch.Tensor,
        values: torch.Tensor,
        gamma: torch.Tensor | float = 0.0,
        init_ram: tuple[torch.Tensor | None, torch.Tensor | float | None] | None = None,
        mask: torch.Tensor | None = None,
        embed_num: int = 0,
        position_ids: torch.Tensor | None = None,
        top_k: tuple[int, int] | list[int] | int | None = 8,
        top_k_re_norm: float | tuple[float, float] | list[float] = 0.0,
        mass_aware: bool = False,
        eps: float = 1e-12,
        t_dim: int = 1,
        inplace: bool = False,
        impl_backend: Literal['torch', 'triton', 'cuda'] | None = None,
) -> tuple[torch.Tensor, tuple[torch.Tensor, torch.Tensor]]:
    """Random-access memory attention.

    :param w_addr: Write address logits (..., T, ..., H, U, P).
    :param r_addr: Read address logits (..., T, ..., H, U, P).
    :param values: Values to write (..., T, ..., H, C).
    :param gamma: Forget-rate control (..., T, ..., H) or a scalar; < 0 remembers, > 0 forgets.
    :param init_ram: Previous ``(slot, mass)``; slot may be None, mass a tensor, scalar or None (1 / A).
    :param mask: Valid-token mask broadcastable to the positions; masked tokens neither write nor read (y = 0).
    :param embed_num: Heads ``h < embed_num`` use CAPE.
    :param position_ids: Token positions broadcastable to (..., T, ...); default ``arange(T)``.
    :param top_k: Kept write/read slots: an int or a ``(write_k, read_k)`` pair.
    :param top_k_re_norm: r in [0, 1] (or a write/read pair); kept q become q / sum(q) ** r.
    :param mass_aware: Weight reads by the updated slot mass.
    :param eps: Strictly positive stabiliser.
    :param t_dim: Index of the time dimension.
    :param inplace: Update the ``init_ram`` tensors in place (contiguous float32 state required).
    :param impl_backend: 'cuda' (HIP) or None.
    :return: ``(y, (slot, mass))`` with shapes (..., T, ..., H, C), (..., H, A, C), (..., H, A).
    """
    assert all(isinstance(t, torch.Tensor) for t in (r_addr, w_addr, values)), \
        f"Expected r_addr/w_addr/values to be tensors, got {type(r_addr).__name__}, {type(w_addr).__name__}, {type(values).__name__}."

    if init_ram is None:
        init_slot, init_mass = None, None
    elif isinstance(init_ram, tuple) and len(init_ram) == 2:
        init_slot, init_mass = init_ram
    else:
        raise TypeError("init_ram must be a (slot, mass) tuple or None.")

    # -- argument types
    assert init_slot is None or isinstance(init_slot, torch.Tensor), f"Expected init_slot to be Tensor or None, got {type(init_slot).__name__}."
    assert init_mass is None or isinstance(init_mass, (torch.Tensor, int, float)), f"Expected init_mass to be Tensor, scalar, or None, got {type(init_mass).__name__}."
    assert isinstance(gamma, (torch.Tensor, int, float)), f"Expected gamma to be Tensor or scalar, got {type(gamma).__name__}."
    assert position_ids is None or isinstance(position_ids, torch.Tensor), f"Expected position_ids to be Tensor or None, got {type(position_ids).__name__}."
    assert mask is None or isinstance(mask, torch.Tensor), f"Expected mask to be Tensor or None, got {type(mask).__name__}."
    assert isinstance(t_dim, int), f"Expected t_dim to be int, got {type(t_dim).__name__}."
    assert isinstance(embed_num, int) and embed_num >= 0, f"Expected embed_num >= 0, got {embed_num!r}."
    assert isinstance(eps, (int, float)) and eps > 0, f"Expected eps > 0, got {eps!r}."
    assert isinstance(mass_aware, bool), f"Expected mass_aware to be bool, got {type(mass_aware).__name__}."
    assert not inplace or isinstance(init_slot, torch.Tensor) and isinstance(init_mass, torch.Tensor), \
        f"inplace=True requires Tensor state, got slot={type(init_slot).__name__}, mass={type(init_mass).__name__}."

    # -- ranks
    for name, tensor, min_ndim in (("w_addr", w_addr, 4), ("r_addr", r_addr, 4), ("values", values, 3)):
        assert tensor.ndim >= min_ndim, f"Expected {name}.ndim >= {min_ndim}, got shape={tuple(tensor.shape)}."
    for name, tensor, min_ndim in (("gamma", gamma, 2), ("init_slot", init_slot, 3), ("init_mass", init_mass, 2),
                                   ("position_ids", position_ids, 1), ("mask", mask, 1)):
        assert not isinstance(tensor, torch.Tensor) or tensor.ndim >= min_ndim, \
            f"Expected {name}.ndim >= {min_ndim}, got shape={tuple(tensor.shape)}."

    # -- the time dimension must sit before each tensor's trailing feature dims
    timed = [("w_addr", w_addr, 3), ("r_addr", r_addr, 3), ("values", values, 2)]
    timed += [(n, t, k) for n, t, k in (("gamma", gamma, 1), ("position_ids", position_ids, 0), ("mask", mask, 0))
              if isinstance(t, torch.Tensor)]
    for name, tensor, trailing in timed:
        assert -tensor.ndim <= t_dim < tensor.ndim and t_dim % tensor.ndim < tensor.ndim - trailing, \
            f"t_dim={t_dim} does not select the time dimension of {name} with shape {tuple(tensor.shape)}."

    # -- dtypes
    assert w_addr.is_floating_point() and r_addr.is_floating_point() and values.is_floating_point(), \
        f"Expected floating-point addresses/values, got {w_addr.dtype=}, {r_addr.dtype=}, {values.dtype=}."
    assert w_addr.dtype == r_addr.dtype == values.dtype, f"Expected matching dtypes, got {w_addr.dtype=}, {r_addr.dtype=}, {values.dtype=}."
    assert not isinstance(gamma, torch.Tensor) or gamma.dtype == values.dtype, f"Expected gamma.dtype={values.dtype}, got {gamma.dtype}."

    # -- time axis last: addresses (..., H, U, P, T), values (..., H, T, C)
    w_addr = w_addr.movedim(t_dim, -1)
    r_addr = r_addr.movedim(t_dim, -1)
    values = values.movedim(t_dim, -2)
    if isinstance(gamma, torch.Tensor):
        gamma = gamma.movedim(t_dim, -1)
    if isinstance(position_ids, torch.Tensor):
        position_ids = position_ids.movedim(t_dim, -1)
    if isinstance(mask, torch.Tensor):
        mask = mask.movedim(t_dim, -1)

    # -- broadcast sizes
    def shape_or(t, default):
        return tuple(t.shape) if isinstance(t, torch.Tensor) else default

    slot_shape, mass_shape = shape_or(init_slot, (1, 1, 1)), shape_or(init_mass, (1, 1))
    gamma_shape, pos_shape, mask_shape = shape_or(gamma, (1, 1)), shape_or(position_ids, (1,)), shape_or(mask, (1,))
    batch_shape = torch.broadcast_shapes(w_addr.shape[:-4], r_addr.shape[:-4], values.shape[:-3], gamma_shape[:-2],
                                         slot_shape[:-3], mass_shape[:-2], pos_shape[:-1], mask_shape[:-1])
    H = get_broadcast(w_addr.size(-4), r_addr.size(-4), values.size(-3), gamma_shape[-2], slot_shape[-3], mass_shape[-2])
    U = get_broadcast(w_addr.size(-3), r_addr.size(-3))
    P = get_broadcast(w_addr.size(-2), r_addr.size(-2))
    A = get_broadcast(slot_shape[-2], mass_shape[-1], P ** U)
    C = get_broadcast(values.size(-1), slot_shape[-1])
    T = get_broadcast(w_addr.size(-1), r_addr.size(-1), values.size(-2), gamma_shape[-1], pos_shape[-1], mask_shape[-1])
    assert all(size > 0 for size in (H, U, P, A, C, T)), f"RAM dimensions must be positive, got {H=}, {U=}, {P=}, {A=}, {C=}, {T=}."
    assert embed_num <= H, f"embed_num must not exceed H={H}, but got {embed_num}."
    if inplace:
        want_slot, want_mass = (*batch_shape, H, A, C), (*batch_shape, H, A)
        assert tuple(init_slot.shape) == want_slot and tuple(init_mass.shape) == want_mass, \
            f"inplace=True expects slot.shape={want_slot}, mass.shape={want_mass}; got {tuple(init_slot.shape)} and {tuple(init_mass.shape)}."
        assert init_slot.is_contiguous() and init_mass.is_contiguous(), \
            f"inplace=True requires contiguous init_ram tensors, got slot{init_slot.is_contiguous()=} and mass{init_mass.is_contiguous()=}."

    # -- defaults: gamma scalar, zero slots, mass 1/A, positions arange(T)
    if not isinstance(gamma, torch.Tensor):
        gamma = values.new_full((*batch_shape, H, 1), fill_value=gamma).expand(*batch_shape, H, T)
    if not isinstance(init_slot, torch.Tensor):
        init_slot = values.new_zeros(*batch_shape, H, A, C)
    if not isinstance(init_mass, torch.Tensor):
        init_mass = values.new_full((*batch_shape, H, A), fill_value=1.0 / (P ** U) if init_mass is None else init_mass)
    if isinstance(position_ids, torch.Tensor):
        position_ids = position_ids.to(device=values.device)
    else:
        position_ids = torch.arange(T, device=values.device, dtype=torch.long).view(*([1] * len(batch_shape)), T)
    if isinstance(mask, torch.Tensor):
        mask = mask.to(device=values.device, dtype=torch.bool)

    # -- broadcast to full shapes and check
    full = {
        "w_addr": (*batch_shape, H, U, P, T), "r_addr": (*batch_shape, H, U, P, T), "values": (*batch_shape, H, T, C),
        "gamma": (*batch_shape, H, T), "init_slot": (*batch_shape, H, A, C), "init_mass": (*batch_shape, H, A),
        "position_ids": (*batch_shape, T),
    }
    w_addr, r_addr = w_addr.broadcast_to(full["w_addr"]), r_addr.broadcast_to(full["r_addr"])
    values, gamma = values.broadcast_to(full["values"]), gamma.broadcast_to(full["gamma"])
    init_slot, init_mass = init_slot.broadcast_to(full["init_slot"]), init_mass.broadcast_to(full["init_mass"])
    position_ids = position_ids.broadcast_to(full["position_ids"])
    if isinstance(mask, torch.Tensor):
        mask = mask.broadcast_to((*batch_shape, T))
    devices = {t.device for t in (w_addr, r_addr, values, gamma, init_slot, init_mass, position_ids)}
    assert len(devices) == 1, f"Expected one device, got {sorted(str(d) for d in devices)}."
    assert mask is None or mask.device == position_ids.device, f"Expected mask.device={position_ids.device}, got {mask.device}."
    for name, tensor in (("w_addr", w_addr), ("r_addr", r_addr), ("values", values), ("gamma", gamma),
                         ("init_slot", init_slot), ("init_mass", init_mass), ("position_ids", position_ids)):
        assert tuple(tensor.shape) == full[name], f"Expected {name}.shape == {full[name]}, but got {tuple(tensor.shape)}."

    # -- flatten the broadcast batch dims into B
    w_addr, r_addr = w_addr.reshape(-1, H, U, P, T), r_addr.reshape(-1, H, U, P, T)
    values, gamma = values.reshape(-1, H, T, C), gamma.reshape(-1, H, T)
    init_slot, init_mass = init_slot.reshape(-1, H, A, C), init_mass.reshape(-1, H, A)
    position_ids = position_ids.reshape(-1, T)
    if isinstance(mask, torch.Tensor):
        mask = mask.reshape(-1, T)

    # -- top-k and re-norm pairs
    if top_k is not None:
        top_k = _as_pair(top_k, int, "`top_k` must be int, a two-item tuple/list of ints, or None.")
        assert all(0 < k <= P ** U for k in top_k), f"top_k values must be in the range (0, {P ** U}], but got {top_k}"
    re_msg = "`top_k_re_norm` must be a number or a two-item tuple/list of numbers in [0, 1]."
    top_k_re_norm = _as_pair(top_k_re_norm, (int, float), re_msg)
    if not all(0 <= v <= 1 for v in top_k_re_norm):
        raise ValueError("`top_k_re_norm` exponents must be in [0, 1].")
    top_k_re_norm = tuple(float(v) for v in top_k_re_norm)

    # -- backend
    if impl_backend not in (None, 'torch', 'triton', 'cuda'):
        raise ValueError(f"Unsupported impl_backend: {impl_backend!r}.")
    if impl_backend == 'torch':
        raise _no_torch_backend("random_access_memory_attention")
    if impl_backend == 'triton':
        raise ValueError("impl_backend='triton' is not available; this package runs on the MI355X HIP backend.")
    if _cuda_ram_attn is None:
        raise _unavailable("random_access_memory_attention")
    if not values.is_cuda or values.dtype not in _HIP_DTYPES or top_k is None:
        raise RuntimeError(
            "random_access_memory_attention on MI355X needs GPU tensors in float16/bfloat16/float32 and top-K mode "
            f"(got {values.dtype} on {values.device}, top_k={top_k}).")

    y, slot, mass = _cuda_ram_attn(w_addr, r_addr, values, gamma, init_slot, init_mass, mask, embed_num,
                                   position_ids, top_k, top_k_re_norm, mass_aware, eps, inplace)

    y = y.reshape(*batch_shape, H, T, C).movedim(-2, t_dim)
    return y, (slot.reshape(*batch_shape, H, A, C), mass.reshape(*batch_shape, H, A))

"""Seeded synthetic inputs for the parity tests and the benchmark.

Inputs are built on the CPU from a ``torch.Generator`` so that the GPU path
and the CPU oracle see identical values. Address logits come either directly
from N(0, 1) (operator tests, like the reference's make_ram_case,
tests/ops/ram_attention_helpers.py:46-94) or from a per-head projection of
q/k (the benchmark configurations: logits = q @ W / sqrt(U) with
W ~ N(0, 1/d_k)).
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import torch


@dataclass
class RamCase:
    w_addr: torch.Tensor      # (B, H, U, P, T)
    r_addr: torch.Tensor      # (B, H, U, P, T)
    values: torch.Tensor      # (B, H, T, C)
    gamma: torch.Tensor       # (B, H, T)
    init_slot: torch.Tensor   # (B, H, A, C) float32
    init_mass: torch.Tensor   # (B, H, A) float32
    position_ids: torch.Tensor  # (B, T) int64
    mask: torch.Tensor | None   # (B, T) bool

    @property
    def shape(self):
        B, H, U, P, T = self.w_addr.shape
        return B, H, U, P, T, self.values.shape[-1]

    def to(self, device, dtype=None):
        def mv(t, cast=True):
            if t is None:
                return None
            t = t.to(device)
            return t.to(dtype) if (dtype is not None and cast) else t
        return RamCase(mv(self.w_addr), mv(self.r_addr), mv(self.values), mv(self.gamma),
                       mv(self.init_slot, False), mv(self.init_mass, False), mv(self.position_ids, False),
                       mv(self.mask, False))


def make_case(B=2, H=4, U=2, P=4, T=33, C=16, dtype=torch.float32, seed=0, masked=False, gamma_scale=0.2,
              gamma_sigmoid_shift=None, random_state=True, quantize=None) -> RamCase:
    """Random operator inputs. ``gamma_sigmoid_shift`` switches gamma to sigmoid(N(0,1) + shift)."""
    g = torch.Generator().manual_seed(seed)
    A = P ** U
    w = torch.randn(B, H, U, P, T, generator=g)
    r = torch.randn(B, H, U, P, T, generator=g)
    if quantize:
        w = torch.round(w / quantize) * quantize
        r = torch.round(r / quantize) * quantize
    x = torch.randn(B, H, T, C, generator=g)
    if gamma_sigmoid_shift is None:
        gamma = gamma_scale * torch.randn(B, H, T, generator=g)
    else:
        gamma = torch.sigmoid(torch.randn(B, H, T, generator=g) + gamma_sigmoid_shift)
    if random_state:
        slot = torch.randn(B, H, A, C, generator=g)
        mass = torch.rand(B, H, A, generator=g) + 0.1
    else:
        slot = torch.zeros(B, H, A, C)
        mass = torch.full((B, H, A), 1.0 / A)
    if masked:
        mask = torch.ones(B, T, dtype=torch.bool)
        pad = max(1, T // 8)
        mid = T // 2 - pad // 2
        mask[:, :pad] = False
        mask[:, mid:mid + pad] = False
        mask[:, -pad:] = False
        pos = (mask.long().cumsum(-1) - 1).masked_fill(~mask, 0)
    else:
        mask = None
        pos = torch.arange(T).view(1, T).expand(B, T).contiguous()
    return RamCase(w.to(dtype), r.to(dtype), x.to(dtype), gamma.to(dtype), slot, mass, pos, mask)


def projected_logits(B, H, U, P, T, d_k, seed, dtype=torch.bfloat16, device="cpu"):
    """Config logits: q, k ~ N(0, 1) of width d_k projected per head to U*P logits (x 1/sqrt(U))."""
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(H, d_k, U * P, generator=g) / d_k ** 0.5
    out = []
    for _ in range(2):  # write (k) then read (q)
        q = torch.randn(B, H, T, d_k, generator=g)
        lg = torch.einsum('bhtd,hdn->bhtn', q, W) / U ** 0.5  # (B, H, T, U*P)
        out.append(lg.view(B, H, T, U, P).permute(0, 1, 3, 4, 2).contiguous().to(dtype).to(device))
    return out[0], out[1]


def with_mask(case: RamCase, mask: torch.Tensor) -> RamCase:
    pos = (mask.long().cumsum(-1) - 1).masked_fill(~mask, 0)
    return replace(case, mask=mask, position_ids=pos)

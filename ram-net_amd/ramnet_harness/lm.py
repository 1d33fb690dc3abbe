"""A RAM-Net decoder-only language model over ``ramnet_ops`` (config 5).

Layer stack, as the reference's block composes it
(``modeling_ramnet.py:18-120``, ``ram_attn_block.py:127-350``):

    x -> x + RamLayer(RMSNorm(x)) -> x + SwiGLU(RMSNorm(x))

RamLayer (the operator's caller):
  * write / read address logits: Linear(d, H*U*P, bias) per head and digit,
    times exp(scale[h, u]) / temperature (temperature sqrt(U) by default,
    ``ram_attn_block.py:300-302``);
  * values: Linear(d, H*C); forget control gamma: Linear(d, H) (the
    'dynamic' mode, ``:305-309``);
  * the operator ``random_access_memory_attention`` with the layer's
    (slot, mass) state, in place for decode steps;
  * head-wise RMSNorm of the read-out, a sigmoid output gate
    Linear(d, H*C), and the output projection Linear(H*C, d) (``:326-334``).

Initialisation follows ``ram_attn_block.py:154-190``: weights N(0, 0.02),
address biases form the prior linspace(0, 1.5, U) x linspace(-1, 1, P), the
gate bias is 3, other biases and the address scales are zero.

The SwiGLU width is an input (FLA's GatedMLP is not available here; 2816 is
its rounding of 8/3 * 1024 to a multiple of 256 and is used for config 5).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn as nn
import torch.nn.functional as F

from ramnet_ops import random_access_memory_attention


@dataclass
class HarnessConfig:
    vocab: int = 32000
    layers: int = 24
    d_model: int = 1024
    heads: int = 8
    value_chs: int = 128
    addr_order: int = 2      # U
    addr_radix: int = 32     # P (A = P ** U = 1024)
    top_k: int = 8
    embed_num: int = 4       # CAPE heads (must be <= heads)
    mlp_width: int = 2816
    gamma: float = 0.0
    norm_eps: float = 1e-6
    ram_eps: float = 1e-12
    dtype: torch.dtype = torch.bfloat16
    extra: dict = field(default_factory=dict)

    @property
    def slots(self) -> int:
        return self.addr_radix ** self.addr_order


class RamLayer(nn.Module):
    """The operator's caller: projections, scaling, gamma, read-out norm and gate."""

    def __init__(self, cfg: HarnessConfig):
        super().__init__()
        if not 0 <= cfg.embed_num <= cfg.heads:
            raise ValueError(f"embed_num must be in [0, {cfg.heads}], got {cfg.embed_num}")
        H, U, P, C, d = cfg.heads, cfg.addr_order, cfg.addr_radix, cfg.value_chs, cfg.d_model
        self.cfg = cfg
        self.w_addr = nn.Linear(d, H * U * P)
        self.r_addr = nn.Linear(d, H * U * P)
        self.value = nn.Linear(d, H * C, bias=False)
        self.gamma = nn.Linear(d, H)
        self.gate = nn.Linear(d, H * C)
        self.out = nn.Linear(H * C, d, bias=False)
        self.out_norm = nn.RMSNorm(C, eps=cfg.norm_eps)
        self.w_scale = nn.Parameter(torch.zeros(H, U))
        self.r_scale = nn.Parameter(torch.zeros(H, U))
        self.temperature = math.sqrt(U)

    @torch.no_grad()
    def init_weights(self, std: float = 0.02, prior: float = 1.5, gate_bias: float = 3.0) -> None:
        H, U, P = self.cfg.heads, self.cfg.addr_order, self.cfg.addr_radix
        for lin in (self.w_addr, self.r_addr, self.value, self.gamma, self.gate, self.out):
            nn.init.normal_(lin.weight, 0.0, std)
        digit_prior = torch.linspace(0, prior, U).view(U, 1) * torch.linspace(-1, 1, P).view(1, P)
        for lin in (self.w_addr, self.r_addr):
            lin.bias.copy_(digit_prior.expand(H, U, P).reshape(-1))
        nn.init.zeros_(self.gamma.bias)
        nn.init.constant_(self.gate.bias, gate_bias)
        nn.init.zeros_(self.w_scale)
        nn.init.zeros_(self.r_scale)

    def op_inputs(self, x: torch.Tensor):
        """(w_addr, r_addr, values, gamma) in the operator's (B, T, H, ...) layout."""
        B, T, _ = x.shape
        H, U, P, C = self.cfg.heads, self.cfg.addr_order, self.cfg.addr_radix, self.cfg.value_chs
        ws = (self.w_scale.exp() / self.temperature).to(x.dtype).unsqueeze(-1)
        rs = (self.r_scale.exp() / self.temperature).to(x.dtype).unsqueeze(-1)
        w = self.w_addr(x).view(B, T, H, U, P) * ws
        r = self.r_addr(x).view(B, T, H, U, P) * rs
        v = self.value(x).view(B, T, H, C)
        g = self.gamma(x) + self.cfg.gamma
        return w, r, v, g

    def forward(self, x: torch.Tensor, state, position_ids: torch.Tensor, inplace: bool, capture=None):
        w, r, v, g = self.op_inputs(x)
        if capture is not None:
            capture.append({"w": w, "r": r, "v": v, "g": g, "pos": position_ids,
                            "slot": state[0].clone() if state[0] is not None else None,
                            "mass": state[1].clone() if isinstance(state[1], torch.Tensor) else state[1]})
        y, new_state = random_access_memory_attention(
            w, r, v, g, init_ram=state, embed_num=self.cfg.embed_num, position_ids=position_ids,
            top_k=self.cfg.top_k, eps=self.cfg.ram_eps, t_dim=1, inplace=inplace, impl_backend="cuda")
        if capture is not None:
            capture[-1]["y"] = y
        y = self.out_norm(y).flatten(-2)
        return self.out(torch.sigmoid(self.gate(x)) * y), new_state


class SwiGLU(nn.Module):
    def __init__(self, d: int, width: int):
        super().__init__()
        self.gate_up = nn.Linear(d, 2 * width, bias=False)
        self.down = nn.Linear(width, d, bias=False)

    def forward(self, x):
        gate, up = self.gate_up(x).chunk(2, dim=-1)
        return self.down(F.silu(gate) * up)


class Block(nn.Module):
    def __init__(self, cfg: HarnessConfig):
        super().__init__()
        self.ram_norm = nn.RMSNorm(cfg.d_model, eps=cfg.norm_eps)
        self.ram = RamLayer(cfg)
        self.mlp_norm = nn.RMSNorm(cfg.d_model, eps=cfg.norm_eps)
        self.mlp = SwiGLU(cfg.d_model, cfg.mlp_width)

    def forward(self, x, state, position_ids, inplace, capture=None):
        h, state = self.ram(self.ram_norm(x), state, position_ids, inplace, capture)
        x = x + h
        return x + self.mlp(self.mlp_norm(x)), state


class RamLM(nn.Module):
    def __init__(self, cfg: HarnessConfig):
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab, cfg.d_model)
        self.blocks = nn.ModuleList(Block(cfg) for _ in range(cfg.layers))
        self.norm = nn.RMSNorm(cfg.d_model, eps=cfg.norm_eps)
        self.head = nn.Linear(cfg.d_model, cfg.vocab, bias=False)

    @torch.no_grad()
    def init_weights(self, std: float = 0.02) -> None:
        nn.init.normal_(self.embed.weight, 0.0, std)
        nn.init.normal_(self.head.weight, 0.0, std)
        for blk in self.blocks:
            blk.ram.init_weights(std)
            nn.init.normal_(blk.mlp.gate_up.weight, 0.0, std)
            nn.init.normal_(blk.mlp.down.weight, 0.0, std)

    def fresh_state(self, batch: int, device) -> list:
        """Per layer (slot, mass): zeros and 1/A, the operator's defaults."""
        cfg = self.cfg
        shape = (batch, cfg.heads, cfg.slots)
        return [(torch.zeros(*shape, cfg.value_chs, device=device), torch.full(shape, 1.0 / cfg.slots, device=device))
                for _ in range(cfg.layers)]

    def forward(self, tokens: torch.Tensor, states: list, position_ids: torch.Tensor, inplace: bool, capture=None):
        x = self.embed(tokens)
        out_states = []
        for blk, st in zip(self.blocks, states):
            x, st = blk(x, st, position_ids, inplace, capture)
            out_states.append(st)
        return self.head(self.norm(x)), out_states


@torch.no_grad()
def greedy_generate(model: RamLM, prompt: torch.Tensor, new_tokens: int, step_hook=None):
    """Prefill ``prompt`` (B, T) with fresh states, then ``new_tokens`` greedy
    single-token steps whose states are updated in place. Returns the
    generated ids (B, new_tokens) and the final states."""
    B, T = prompt.shape
    dev = prompt.device
    states = model.fresh_state(B, dev)
    pos = torch.arange(T, device=dev).view(1, T).expand(B, T)
    logits, states = model(prompt, states, pos, inplace=False)
    tok = logits[:, -1].argmax(-1, keepdim=True)
    out = [tok]
    for s in range(1, new_tokens):
        p = torch.full((B, 1), T + s - 1, device=dev, dtype=torch.long)
        logits, states = model(tok, states, p, inplace=True)
        tok = logits[:, -1].argmax(-1, keepdim=True)
        out.append(tok)
        if step_hook is not None:
            step_hook(s)
    return torch.cat(out, dim=1), states

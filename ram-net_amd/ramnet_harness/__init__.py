"""Config-5 caller harness: a RAM-Net language model above the operator.

Not part of the operator library. It exercises ``ramnet_ops`` the way the
reference's model does (``packages/ramnet``: ``ram_attn_block.py:281-350``,
``modeling_ramnet.py:71-107``): a prefill over a prompt with a fresh state,
then greedy single-token steps that update each layer's state in place.
"""
from .lm import HarnessConfig, RamLM, RamLayer, greedy_generate

__all__ = ["HarnessConfig", "RamLM", "RamLayer", "greedy_generate"]

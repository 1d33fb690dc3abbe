"""RAM-Net operators on AMD MI355X (gfx950).

Drop-in for the reference ``ramnet_ops`` package
(packages/ramnet-ops/src/ramnet_ops/__init__.py:1-6): the same two public
functions, computed by hand-written HIP kernels through a C ABI.
"""
from .ram_attn import random_access_memory_attention, topk_addr

__all__ = [
    'random_access_memory_attention',
    'topk_addr',
]

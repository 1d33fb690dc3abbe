"""Index-width limits of the device kernels (reference: impl/_cuda_config.py:1-11).

``INT_BITS`` comes from the C ABI (``ramnet_int_bits``). Addresses keep one
spare magnitude bit for intermediate index arithmetic.
"""
from .. import _native

INT_BITS = _native.int_bits()
INT_MAX = (1 << (INT_BITS - 1)) - 1
ADDRESS_LIMIT = 1 << (INT_BITS - 2)


def check_int_capacity(*sizes: int) -> None:
    """Every size and size product handed to the kernels must fit a signed int32."""
    assert all(0 <= size < INT_MAX for size in sizes), f"CUDA index overflow: sizes={sizes}, limit={INT_MAX}."

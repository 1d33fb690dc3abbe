"""Backends of ``ramnet_ops``: the gfx950 HIP operators (``cuda_impl``)."""

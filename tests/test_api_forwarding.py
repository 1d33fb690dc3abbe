"""Public API option handling and forwarding, with the backend mocked.

Mirrors the reference's API tests (tests/ops/test_ram_attention_api.py:
14-160): ``mass_aware`` and the normalised ``top_k_re_norm`` pair reach the
backend unchanged, invalid ``top_k_re_norm`` values raise ``TypeError`` or
``ValueError`` naming the option before any backend call, the decoder
forwards its options as given, and an unknown or unavailable backend raises.
Differences by design: ``impl_backend='torch'`` (the reference's CPU path)
is not part of this package, and the HIP path refuses CPU tensors before
dispatch, so the forwarding checks use GPU tensors.
"""
from __future__ import annotations

from unittest.mock import patch

import pytest
import torch


def _api():
    import ramnet_ops.ram_attn as api
    return api


def _fake_ram_attn(seen):
    def fake(w_addr, r_addr, x, gamma, init_slot, init_mass, mask, embed_num, position_ids, top_k, top_k_re_norm,
             mass_aware, eps, inplace):
        seen.update(top_k=top_k, top_k_re_norm=top_k_re_norm, mass_aware=mass_aware, eps=eps, inplace=inplace)
        return x, init_slot, init_mass
    return fake


INVALID_TYPE = (None, "0.5", [0.5], (0.0, 0.5, 1.0), (0.5, None))
INVALID_VALUE = (-0.1, 1.1, float("nan"), float("inf"), -float("inf"), (0.0, 1.1), (float("nan"), 0.5))


def test_re_norm_rejects_invalid_values_before_the_backend():
    api = _api()
    addr = torch.zeros(1, 1, 1, 1, 16)
    values = torch.zeros(1, 1, 1, 4)
    with patch.object(api, "_cuda_ram_attn") as impl:
        for option in INVALID_TYPE:
            with pytest.raises(TypeError, match="top_k_re_norm"):
                api.random_access_memory_attention(addr, addr, values, top_k_re_norm=option, impl_backend="cuda")
        for option in INVALID_VALUE:
            with pytest.raises(ValueError, match="top_k_re_norm"):
                api.random_access_memory_attention(addr, addr, values, top_k_re_norm=option, impl_backend="cuda")
        impl.assert_not_called()
    addr = torch.zeros(1, 1, 1, 2, 1)
    pos = torch.zeros(1, 1, dtype=torch.long)
    with patch.object(api, "_cuda_topk_addr") as impl:
        for option, error in ((None, TypeError), ("0.5", TypeError), ((0.25, 0.75), TypeError), (-0.1, ValueError),
                              (1.1, ValueError), (float("nan"), ValueError), (float("inf"), ValueError),
                              (-float("inf"), ValueError)):
            with pytest.raises(error, match="top_k_re_norm"):
                api.topk_addr(addr, 0, pos, 1, option, impl_backend="cuda")
        impl.assert_not_called()


def test_invalid_or_unavailable_backend():
    api = _api()
    addr = torch.zeros(1, 1, 1, 2, 1)
    pos = torch.zeros(1, 1, dtype=torch.long)
    with pytest.raises(ValueError, match="impl_backend"):
        api.topk_addr(addr, 0, pos, 1, 0.0, impl_backend="invalid")
    with patch.object(api, "_cuda_topk_addr", None):
        with pytest.raises(RuntimeError, match="could not be loaded"):
            api.topk_addr(addr, 0, pos, 1, 0.0, impl_backend="cuda")
    values = torch.zeros(1, 1, 1, 4)
    with patch.object(api, "_cuda_ram_attn", None):
        with pytest.raises(RuntimeError, match="could not be loaded"):
            api.random_access_memory_attention(torch.zeros(1, 1, 1, 2, 1), torch.zeros(1, 1, 1, 2, 1), values, top_k=1)


@pytest.mark.gpu
@pytest.mark.parametrize("mass_aware", [False, True])
def test_mass_aware_reaches_backend(mass_aware):
    api = _api()
    addresses = torch.zeros(1, 2, 1, 1, 8, device="cuda")
    values = torch.zeros(1, 2, 1, 4, device="cuda")
    seen = {}
    with patch.object(api, "_cuda_ram_attn", side_effect=_fake_ram_attn(seen)) as impl:
        api.random_access_memory_attention(addresses, addresses, values, top_k=1, mass_aware=mass_aware,
                                           impl_backend="cuda")
    impl.assert_called_once()
    assert seen["mass_aware"] is mass_aware


@pytest.mark.gpu
@pytest.mark.parametrize("option,expected", [(0.0, (0.0, 0.0)), (0.5, (0.5, 0.5)), (1.0, (1.0, 1.0)),
                                             ((0.25, 0.75), (0.25, 0.75)), ([0.75, 0.25], (0.75, 0.25)),
                                             ((0, 1), (0.0, 1.0)), (True, (1.0, 1.0)), (False, (0.0, 0.0))])
def test_re_norm_preserves_explicit_values(option, expected):
    api = _api()
    addr = torch.zeros(1, 1, 1, 1, 16, device="cuda")
    values = torch.zeros(1, 1, 1, 4, device="cuda")
    seen = {}
    with patch.object(api, "_cuda_ram_attn", side_effect=_fake_ram_attn(seen)):
        api.random_access_memory_attention(addr, addr, values, top_k=(4, 12), top_k_re_norm=option,
                                           impl_backend="cuda")
    assert seen["top_k_re_norm"] == expected and all(type(v) is float for v in seen["top_k_re_norm"])
    assert seen["top_k"] == (4, 12)


@pytest.mark.gpu
def test_topk_addr_forwards_options():
    api = _api()
    from ramnet_ops import topk_addr
    assert topk_addr is api.topk_addr
    addr = torch.zeros(2, 2, 2, 3, 5, device="cuda")
    pos = torch.arange(5, device="cuda").expand(2, -1)
    args = (addr, 1, pos, 4, 0.5, True, False)
    for backend in (None, "cuda"):
        with patch.object(api, "_cuda_topk_addr", return_value=(None, None)) as impl:
            api.topk_addr(*args, impl_backend=backend)
        impl.assert_called_once_with(*args)

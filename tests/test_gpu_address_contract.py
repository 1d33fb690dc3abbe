"""Contracts of the single-address decoder wrapper and of its backward op.

Mirrors the reference's CUDA address tests (tests/ops/test_cuda_address.py:
49-106): the batch-encoded and batch-local indices differ by exactly the
batch offset with identical weights and gradients; indices are int32 without
grad, weights float32, the gradient keeps the logits' dtype and the input is
left unchanged; the registered backward op, called directly, matches
autograd, passes ``opcheck`` and rejects a missing logits tensor. (The
reference's padded-T index limit has no counterpart: T is not padded here.
The address-space limit is tested on meta tensors in test_abi.py.)
"""
from __future__ import annotations

import itertools

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _ops():
    import ramnet_ops  # noqa: F401  (registers torch.ops.ramnet_ops.*)
    return torch.ops.ramnet_ops


def _addr(T, seed):
    g = torch.Generator().manual_seed(seed)
    B, H, U, P = 2, 2, 2, 4
    a = torch.randn(B, H, U, P, T, generator=g)
    pos = torch.arange(T, dtype=torch.int32).view(1, T).expand(B, T).contiguous()
    return a.to(DEV), pos.to(DEV)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("re_norm", [0.0, 0.5, 1.0])
@pytest.mark.parametrize("neg", [False, True])
def test_single_address_wrapper_contract(dtype, re_norm, neg):
    _ops()
    from ramnet_ops.impl.cuda_impl import _cuda_topk_addr
    src, pos = _addr(31, seed=3 + neg)
    addr = src.to(dtype).detach().requires_grad_()
    original = addr.detach().clone()
    idx, val = _cuda_topk_addr(addr, 1, pos, 3, re_norm, neg)
    lidx, lval = _cuda_topk_addr(addr, 1, pos, 3, re_norm, neg, encode_batch_idx=False)
    B, H, U, P, _ = addr.shape
    offset = torch.arange(B, device=DEV, dtype=idx.dtype).view(B, 1, 1, 1) * H * P ** U
    assert torch.equal(idx, lidx + offset)
    assert torch.equal(val, lval)
    assert idx.shape == (2, 2, 3, 31) and idx.dtype == torch.int32 and val.dtype == torch.float32
    assert not idx.requires_grad
    grad = torch.randn_like(val)
    got, = torch.autograd.grad(val, addr, grad)
    local, = torch.autograd.grad(lval, addr, grad)
    assert torch.equal(got, local)
    assert bool(torch.isfinite(val).all()) and bool(torch.isfinite(got).all())
    assert got.dtype == dtype
    assert torch.equal(addr, original)


@pytest.mark.parametrize("re_norm", [0.0, 0.5, 1.0])
@pytest.mark.parametrize("encode_batch_idx", [False, True])
def test_single_address_backward_contract(re_norm, encode_batch_idx):
    ops = _ops()
    src, pos = _addr(32, seed=11)
    addr = src.detach().requires_grad_()
    B, H, U, P, T = addr.shape
    idx, val = ops.topk_addr_single_forward(addr, 1, P ** U, pos, 3, re_norm, encode_batch_idx=encode_batch_idx)
    grad = torch.randn_like(val)
    expected, = torch.autograd.grad(val, addr, grad)
    args = (idx, val.detach(), addr.detach(), grad, 1, pos, 3, re_norm, False, (B, H, U, P, P ** U, T), addr.dtype)
    got = ops.topk_addr_single_backward(*args)
    torch.testing.assert_close(got, expected, atol=1e-5, rtol=1e-5)
    torch.library.opcheck(ops.topk_addr_single_backward, args, test_utils=("test_schema", "test_faketensor"))
    with pytest.raises(RuntimeError):
        ops.topk_addr_single_backward(*args[:2], None, *args[3:])

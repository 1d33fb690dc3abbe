"""Dispatcher schemas, fake tensors, autograd registration and the all-masked
state identity of the ``ramnet_ops`` operators.

Mirrors the reference's registration contract (tests/ops/
test_cuda_registration.py:17-135) with ``torch.library.opcheck``. The
reference's segment operators take its slot-sorted segment metadata; here
``topk_segment_forward`` / ``topk_segment_forward_`` take the decoder's
``(idx, val)`` and the mask directly (the time-ordered scan needs no
segments), so their checks pass those.
"""
from __future__ import annotations

import itertools

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
CHECKS = ("test_schema", "test_autograd_registration", "test_faketensor")


def _ops():
    import ramnet_ops  # noqa: F401  (registers torch.ops.ramnet_ops.*)
    return torch.ops.ramnet_ops


def _case(order=2, T=32, seed=0):
    g = torch.Generator().manual_seed(seed + 17 * order)
    B, H, P, C = 2, 2, 4, 7
    A = P ** order

    def rn(*s):
        return torch.randn(*s, generator=g).to(DEV)

    return dict(w=rn(B, H, order, P, T), r=rn(B, H, order, P, T), x=rn(B, H, T, C), gamma=0.2 * rn(B, H, T),
                slot=rn(B, H, A, C), mass=(torch.rand(B, H, A, generator=g) + 0.1).to(DEV),
                pos=torch.arange(T, dtype=torch.int32, device=DEV).view(1, T).expand(B, T).contiguous(), A=A)


@pytest.mark.parametrize("order", [2, 4])
def test_functional_registrations(order):
    ops = _ops()
    c = _case(order)
    w = c["w"].clone().requires_grad_()
    r = c["r"].clone().requires_grad_()
    A, pos = c["A"], c["pos"]
    torch.library.opcheck(ops.topk_addr_single_forward, (w, 1, A, pos, 2, 0.0), test_utils=CHECKS)
    for (addr, k, re_norm, neg), enc in itertools.product(((w, 2, 0.5, False), (r, 3, 1.0, True)), (False, True)):
        torch.library.opcheck(ops.topk_addr_single_forward, (addr, 1, A, pos, k, re_norm, neg),
                              kwargs={"encode_batch_idx": enc}, test_utils=CHECKS)
    args = (w, r, 1, A, pos, 2, 3, 0.25, 0.75)
    for enc in (False, True):
        torch.library.opcheck(ops.topk_addr_forward, args, kwargs={"encode_batch_idx": enc}, test_utils=CHECKS)
    idx, val = ops.topk_addr_forward(*args)
    mask = torch.ones(2, 32, dtype=torch.bool, device=DEV)
    mask[:, ::5] = False
    for m in (None, mask):
        seg = (idx.detach(), val.detach().requires_grad_(), c["x"].clone().requires_grad_(),
               c["gamma"].clone().requires_grad_(), c["slot"].clone().requires_grad_(),
               c["mass"].clone().requires_grad_(), m, 2, 3, True, 1e-6)
        torch.library.opcheck(ops.topk_segment_forward, seg, test_utils=CHECKS)
    torch.library.opcheck(ops.ram_attn_forward, (c["w"], c["r"], c["x"], c["gamma"], c["slot"], c["mass"], mask, 1,
                                                 pos, 2, 3, 0.25, 0.75, True, 1e-6),
                          test_utils=("test_schema", "test_faketensor"))


def test_inplace_schemas():
    ops = _ops()
    c = _case()
    pos = c["pos"]
    idx, val = ops.topk_addr_forward(c["w"], c["r"], 1, 16, pos, 2, 3, 0.25, 0.75)
    torch.library.opcheck(ops.topk_segment_forward_, (idx, val, c["x"], c["gamma"], c["slot"].clone(),
                                                      c["mass"].clone(), None, 2, 3, True, 1e-6),
                          test_utils=("test_schema", "test_faketensor"))
    torch.library.opcheck(ops.ram_attn_forward_, (c["w"], c["r"], c["x"], c["gamma"], c["slot"].clone(),
                                                  c["mass"].clone(), None, 1, pos, 2, 3, 0.25, 0.75, True, 1e-6),
                          test_utils=("test_schema", "test_faketensor"))
    torch.library.opcheck(ops.topk_autoregressive_, (c["w"][..., 0], c["r"][..., 0], c["x"][..., 0, :],
                                                     c["gamma"][..., 0], c["slot"].clone(), c["mass"].clone(),
                                                     torch.empty(0, dtype=torch.bool, device=DEV), 1, pos[:, 0],
                                                     2, 3, 0.25, 0.75, True, 1e-6),
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.parametrize("order", [2, 4])
def test_all_masked_state_identity(order):
    """Every token masked: y is exactly zero, the post state equals the
    initial state in new storage, and the gradients are zero for the
    addresses, values and gamma and exactly one for the initial state under
    an upstream of ones."""
    _ops()
    from ramnet_ops.impl.cuda_impl import _cuda_ram_attn
    c = _case(order)
    inputs = tuple(t.detach().clone().requires_grad_() for t in (c["w"], c["r"], c["x"], c["gamma"], c["slot"],
                                                                 c["mass"]))
    mask = torch.zeros(2, 32, dtype=torch.bool, device=DEV)
    y, slot, mass = _cuda_ram_attn(*inputs, mask, 1, c["pos"], (2, 3), (0.25, 0.75), True, 1e-6, False)
    assert torch.equal(y, torch.zeros_like(y))
    for got, init in zip((slot, mass), inputs[4:]):
        assert got.data_ptr() != init.data_ptr()
        assert torch.equal(got, init)
    grads = torch.autograd.grad(slot.sum() + mass.sum(), inputs)
    for gr in grads[:4]:
        assert torch.equal(gr, torch.zeros_like(gr))
    for gr in grads[4:]:
        assert torch.equal(gr, torch.ones_like(gr))

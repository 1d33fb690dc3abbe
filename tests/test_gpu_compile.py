"""Fixed-shape ``torch.compile`` and HIP-graph replay of the operators.

Mirrors the reference's compile contract (tests/ops/test_cuda_compile.py:
16-156, tests/compile_helpers.py:10-49): the op glue traces with
``fullgraph=True, dynamic=False`` (every operator has a fake), compiled and
eager runs agree, a repeated shape does not recompile, the captured graph
holds the ``ramnet_ops`` operators, and a captured graph replays with fresh
inputs. Compilation uses the ``aot_eager`` backend (tracing, fake tensors
and the autograd split, without code generation). Graph replay captures the
eager op path on a side stream and replays it three times, each time
against an eager run on new inputs.

The fused no-gradient paths run ``ram_attn_forward`` / ``ram_attn_forward_``
(decoder and scan in one native call) where the reference runs
``topk_segment_forward`` / ``topk_segment_forward_``; the autoregressive step
is ``topk_autoregressive_`` in both.
"""
from __future__ import annotations

from contextlib import contextmanager

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
BACKEND = "aot_eager"


def _impl():
    import ramnet_ops  # noqa: F401  (registers torch.ops.ramnet_ops.*)
    from ramnet_ops.impl import cuda_impl
    return cuda_impl


def _case(order=2, seq_len=32, seed=0):
    """The reference's small CUDA case (tests/ops/cuda_helpers.py:6-10): B=2,
    H=2, radix 4, 7 channels, float32, unmasked positions."""
    g = torch.Generator().manual_seed(seed * 1000 + order * 100 + seq_len)
    B, H, P, C, T = 2, 2, 4, 7, seq_len
    A = P ** order

    def rn(*s):
        return torch.randn(*s, generator=g)

    c = dict(w=rn(B, H, order, P, T), r=rn(B, H, order, P, T), x=rn(B, H, T, C), gamma=0.2 * rn(B, H, T),
             slot=rn(B, H, A, C), mass=torch.rand(B, H, A, generator=g) + 0.1, d_y=rn(B, H, T, C),
             d_slot=rn(B, H, A, C), d_mass=rn(B, H, A),
             pos=torch.arange(T).view(1, T).expand(B, T).contiguous())
    return {k: v.to(DEV) for k, v in c.items()}


def _run(impl, w, r, x, gamma, slot, mass, pos, mask, inplace=False):
    """The reference's call (tests/ops/cuda_helpers.py:13-32): embed_num 1,
    top_k (2, 3), re_norm (0.25, 0.75), mass_aware, eps 1e-6."""
    return impl._cuda_ram_attn(w, r, x, gamma, slot, mass, mask, 1, pos, (2, 3), (0.25, 0.75), True, 1e-6, inplace)


@contextmanager
def _compiled(func):
    from torch._dynamo import config
    from torch._dynamo.testing import CompileCounterWithBackend
    torch.compiler.reset()
    counter = CompileCounterWithBackend(BACKEND)
    try:
        with config.patch(suppress_errors=False):  # a failed compile must not fall back to eager
            yield torch.compile(func, backend=counter, fullgraph=True, dynamic=False), counter
    finally:
        torch.compiler.reset()


def _assert_ops(counter, *names):
    targets = {str(node.target) for graph in counter.graphs for module in graph.modules()
               if isinstance(module, torch.fx.GraphModule) for node in module.graph.nodes}
    for name in names:
        prefix = f"ramnet_ops.{name}"
        assert any(t == prefix or t.startswith(prefix + ".") for t in targets), (name, sorted(targets))


@pytest.mark.parametrize("re_norm", [0.0, 0.5, 1.0])
@pytest.mark.parametrize("encode_batch_idx", [False, True])
def test_compile_single_address_forward_and_backward(re_norm, encode_batch_idx):
    impl = _impl()

    def forward(addr, pos):
        return impl._cuda_topk_addr(addr, 1, pos, 3, re_norm, True, encode_batch_idx=encode_batch_idx)

    with _compiled(forward) as (compiled, counter):
        frames = None
        for i, T in enumerate((32, 33, 33)):
            c = _case(seq_len=T, seed=i)
            results = []
            for fn in (forward, compiled):
                addr = c["r"].detach().clone().requires_grad_()
                idx, val = fn(addr, c["pos"])
                grad, = torch.autograd.grad(val.square().sum(), addr)
                results.append((idx, val, grad))
            ref, got = results
            assert torch.equal(got[0], ref[0])
            for a, b in zip(got[1:], ref[1:]):
                torch.testing.assert_close(a, b, atol=1e-5, rtol=1e-5)
            if i == 2:
                assert counter.frame_count == frames, "a repeated shape recompiled"
            frames = counter.frame_count
        _assert_ops(counter, "topk_addr_single_forward")


@pytest.mark.parametrize("order,state_grad", [(2, False), (4, True)])
def test_compile_parallel_forward_and_backward(order, state_grad):
    impl = _impl()

    def forward(w, r, x, gamma, slot, mass, pos, mask):
        return _run(impl, w, r, x, gamma, slot, mass, pos, mask)

    with _compiled(forward) as (compiled, counter):
        frames = None
        for i, T in enumerate((31, 32, 33, 33)):
            c = _case(order=order, seq_len=T, seed=i)
            mask = torch.ones(2, T, device=DEV, dtype=torch.bool)
            mask[:, ::4] = False
            if i == 3:
                mask[1] = False
            originals = (c["w"], c["r"], c["x"], c["gamma"], c["slot"], c["mass"])
            upstream = (c["d_y"], c["d_slot"], c["d_mass"])
            results = []
            for fn in (forward, compiled):
                inputs = tuple(t.detach().clone().requires_grad_(k < 4 or state_grad) for k, t in enumerate(originals))
                y, slot, mass = fn(*inputs, c["pos"], mask)
                outputs = (y.masked_fill(~mask[:, None, :, None], 0), slot, mass)
                grads = torch.autograd.grad(outputs, inputs if state_grad else inputs[:4], upstream)
                results.append((*outputs, *grads))
                for cur, orig in zip(inputs[4:], originals[4:]):
                    assert torch.equal(cur, orig), "the functional form changed its initial state"
            ref, got = results
            for a, b in zip(got, ref):
                torch.testing.assert_close(a, b, atol=5e-4, rtol=5e-4)
            if i == 3:
                assert counter.frame_count == frames, "a repeated shape recompiled"
            frames = counter.frame_count
        _assert_ops(counter, "topk_addr_forward", "topk_segment_forward")


@pytest.mark.parametrize("seq_len", [1, 33], ids=["autoregressive", "parallel"])
def test_compile_inplace(seq_len):
    impl = _impl()
    c0 = _case(seq_len=seq_len)
    ref_slot, ref_mass = c0["slot"].clone(), c0["mass"].clone()
    slot, mass = c0["slot"].clone(), c0["mass"].clone()

    def forward(w, r, x, gamma, slot, mass, pos, mask):
        return _run(impl, w, r, x, gamma, slot, mass, pos, mask, inplace=True)

    with _compiled(forward) as (compiled, counter):
        frames = None
        for step in range(3):
            c = _case(seq_len=seq_len, seed=step + 1)
            mask = torch.ones(2, seq_len, device=DEV, dtype=torch.bool)
            mask[step % 2, ::2] = False
            pos = c["pos"] + step * seq_len
            ref = forward(c["w"], c["r"], c["x"], c["gamma"], ref_slot, ref_mass, pos, mask)
            got = compiled(c["w"], c["r"], c["x"], c["gamma"], slot, mass, pos, mask)
            assert got[1].data_ptr() == slot.data_ptr() and got[2].data_ptr() == mass.data_ptr()
            for a, b in zip(got, ref):
                torch.testing.assert_close(a, b, atol=5e-4, rtol=5e-4)
            if step:
                assert counter.frame_count == frames, "a repeated shape recompiled"
            frames = counter.frame_count
        _assert_ops(counter, "topk_autoregressive_" if seq_len == 1 else "ram_attn_forward_")


@pytest.mark.parametrize("seq_len,inplace", [(1, True), (33, False), (33, True)])
def test_graph_replay(seq_len, inplace):
    """Capture the op path once, then replay it three times with new inputs
    copied into the captured buffers; every replay matches an eager run, and
    eager work and synchronisation run between the replays."""
    impl = _impl()
    c0 = _case(seq_len=seq_len)
    static = [c0[k].clone() for k in ("w", "r", "x", "gamma", "slot", "mass", "pos")]
    static.append(torch.ones(2, seq_len, device=DEV, dtype=torch.bool))

    def forward(w, r, x, gamma, slot, mass, pos, mask):
        return _run(impl, w, r, x, gamma, slot, mass, pos, mask, inplace=inplace)

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):  # warm-up outside the capture (allocator pools, library load)
            forward(*[t.clone() for t in static])
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        outputs = forward(*static)
    torch.cuda.synchronize()

    for step in range(3):
        c = _case(seq_len=seq_len, seed=step + 7)
        mask = torch.ones(2, seq_len, device=DEV, dtype=torch.bool)
        mask[step % 2, ::2] = False
        inputs = [c[k] for k in ("w", "r", "x", "gamma", "slot", "mass")] + [c["pos"] + step * seq_len, mask]
        for dst, src in zip(static, inputs):
            dst.copy_(src)
        ref = forward(*[t.clone() for t in inputs])
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(outputs, ref):
            torch.testing.assert_close(got, want, atol=5e-4, rtol=5e-4)
        if inplace:
            assert outputs[1].data_ptr() == static[4].data_ptr() and outputs[2].data_ptr() == static[5].data_ptr()
        else:
            assert torch.equal(static[4], c["slot"]) and torch.equal(static[5], c["mass"])

"""``ramnet_ram_attn_forward_noalloc``: the prefill forward with its records
in the library's per-GPU scratch array instead of a caller workspace.

Called through the C ABI and compared with ``ramnet_ram_attn_forward`` (the
same kernels with a caller workspace) on the same inputs: outputs and post
state must be identical bits. Two calls in a row, the second on a smaller
input (the scratch keeps the first call's records, which the second must not
read), then a slot space wide enough for the precomputed-gain form (whose
gain records also live in the scratch), the full config-2 shape (which plans
the precomputed-gain form and needs 162 MiB of the 192 MiB scratch), calls
without tokens or without batch rows, one call captured in a HIP graph and
replayed on fresh inputs, and a shape beyond the scratch, which is refused
on the host before anything is launched.
"""
from __future__ import annotations

import pytest
import torch

from ram_cases import make_case

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _nat():
    import ramnet_ops  # noqa: F401
    from ramnet_ops import _native
    _native.lib()
    return _native


def _launch(nat, d, U, P, K, E, re_norm, mass_aware, noalloc, out=None):
    """One forward call on device inputs ``d`` (a case already on the GPU);
    returns (y, slot, mass), written into ``out`` if given."""
    B, H, _, _, T = d.w_addr.shape
    C = d.values.shape[-1]
    A = P ** U
    pos = d.position_ids.to(torch.int32).contiguous()
    mask = None if d.mask is None else d.mask.to(torch.uint8).contiguous()
    if out is None:
        out = (torch.empty_like(d.values), torch.empty_like(d.init_slot), torch.empty_like(d.init_mass))
    y, slot, mass = out
    code = nat.DTYPE_CODES[d.values.dtype]
    stream = torch.cuda.current_stream().cuda_stream
    args = [d.w_addr.data_ptr(), d.r_addr.data_ptr(), d.values.data_ptr(), d.gamma.data_ptr(), code, nat.ptr(mask), E,
            pos.data_ptr(), d.init_slot.data_ptr(), d.init_mass.data_ptr(), slot.data_ptr(), mass.data_ptr(),
            y.data_ptr(), B, H, U, P, T, A, C, K[0], K[1], re_norm[0], re_norm[1], int(mass_aware), 1e-12]
    if noalloc:
        nat.call("ramnet_ram_attn_forward_noalloc", *args, stream)
    else:
        ws = torch.empty(max(1, nat.scan_workspace_bytes(B, H, T, *K)), dtype=torch.uint8, device=DEV)
        nat.call("ramnet_ram_attn_forward", *args, ws.data_ptr(), ws.numel(), stream)
    return out


def _run(nat, case, K, E, re_norm, mass_aware, noalloc):
    U, P = case.shape[2], case.shape[3]
    out = _launch(nat, case.to(DEV), U, P, K, E, re_norm, mass_aware, noalloc)
    torch.cuda.synchronize()
    return tuple(t.cpu() for t in out)


def _same(nat, case, K, E, re_norm, mass_aware, label):
    print(f"no-allocation forward: {label}", flush=True)
    got = _run(nat, case, K, E, re_norm, mass_aware, True)
    want = _run(nat, case, K, E, re_norm, mass_aware, False)
    for name, a, b in zip(("y", "slot", "mass"), got, want):
        assert torch.equal(a, b), f"{label}: {name} differs from ramnet_ram_attn_forward"
    assert bool(torch.isfinite(got[0]).all())


def test_noalloc_matches_workspace_entry_point():
    nat = _nat()
    big = make_case(B=4, H=8, U=2, P=32, T=1024, C=128, dtype=torch.bfloat16, seed=81, masked=True,
                    gamma_sigmoid_shift=-1.0)
    small = make_case(B=2, H=4, U=2, P=16, T=333, C=64, dtype=torch.float32, seed=82, masked=False)
    _same(nat, big, (8, 8), 4, (0.0, 0.0), False, "first call: B=4 H=8 T=1024 A=1024 bf16, masked")
    _same(nat, small, (4, 12), 2, (0.25, 0.75), True, "second call: B=2 H=4 T=333 A=256 fp32, mass_aware")


def test_noalloc_precomputed_gain_form(monkeypatch):
    nat = _nat()
    monkeypatch.setenv("RAMNET_SCAN_LAYOUT", "1,16,1,2,1")
    case = make_case(B=2, H=2, U=3, P=16, T=700, C=64, dtype=torch.bfloat16, seed=83, masked=True)
    assert nat.segment_plan(2, 2, 4096, 64, 8, 8, torch.bfloat16)[2]
    _same(nat, case, (8, 8), 1, (0.0, 0.0), True, "precomputed-gain form: A=4096 T=700")


def test_noalloc_config2_shape():
    """Config 2 (B=8, H=16, T=4096, A=1024, K=8, bf16, CAPE on half the
    heads, zero initial state) plans the precomputed-gain form: 96 MiB of
    decoder records plus 64 MiB of gain records in the scratch."""
    nat = _nat()
    B, H, U, P, T, C, K, E = 8, 16, 2, 32, 4096, 128, 8, 8
    A = P ** U
    assert nat.segment_plan(B, H, A, C, K, K, torch.bfloat16)[2]
    g = torch.Generator(device=DEV).manual_seed(84)
    bf = dict(device=DEV, dtype=torch.bfloat16)
    from ram_cases import RamCase
    d = RamCase(torch.randn(B, H, U, P, T, generator=g, **bf), torch.randn(B, H, U, P, T, generator=g, **bf),
                torch.randn(B, H, T, C, generator=g, **bf),
                torch.sigmoid(torch.randn(B, H, T, generator=g, device=DEV) - 1).to(torch.bfloat16),
                torch.zeros(B, H, A, C, device=DEV), torch.full((B, H, A), 1.0 / A, device=DEV),
                torch.arange(T, device=DEV).view(1, T).expand(B, T).contiguous(), None)
    print("no-allocation forward: config 2, B=8 H=16 T=4096 A=1024 K=8 bf16", flush=True)
    got = _launch(nat, d, U, P, (K, K), E, (0.0, 0.0), False, True)
    want = _launch(nat, d, U, P, (K, K), E, (0.0, 0.0), False, False)
    torch.cuda.synchronize()
    for name, a, b in zip(("y", "slot", "mass"), got, want):
        assert torch.equal(a, b), f"config 2: {name} differs from ramnet_ram_attn_forward"
    assert bool(torch.isfinite(got[0]).all()) and float(got[1].abs().max()) > 0


def test_noalloc_empty_calls():
    """No tokens: the post state is a copy of the initial state, in both scan
    forms (A = 32768 takes the precomputed-gain form in slot ranges). No
    batch rows: nothing to do, and the call succeeds as the workspace entry
    point does."""
    nat = _nat()
    for (U, P, C, K) in ((2, 16, 24, (4, 4)), (3, 32, 16, (8, 8))):
        case = make_case(B=2, H=3, U=U, P=P, T=0, C=C, dtype=torch.bfloat16, seed=85)
        print(f"no-allocation forward: T=0, A={P ** U}", flush=True)
        for noalloc in (True, False):
            y, slot, mass = _run(nat, case, K, 1, (0.0, 0.0), False, noalloc)
            assert y.numel() == 0
            assert torch.equal(slot, case.init_slot) and torch.equal(mass, case.init_mass)
    case = make_case(B=0, H=2, U=2, P=4, T=40, C=8, seed=86)
    print("no-allocation forward: B=0", flush=True)
    y, slot, mass = _run(nat, case, (4, 4), 0, (0.0, 0.0), False, True)
    assert y.numel() == slot.numel() == mass.numel() == 0


def test_noalloc_graph_capture_replays():
    """One call captured in a HIP graph (the library allocates nothing and
    issues no memset), replayed three times on fresh inputs written into the
    captured tensors, with eager work and a synchronisation between the
    replays: every replay is bit-equal to the workspace entry point's eager
    call on the same inputs."""
    nat = _nat()
    B, H, U, P, T, C, K = 2, 4, 2, 16, 300, 64, (8, 8)
    static = make_case(B=B, H=H, U=U, P=P, T=T, C=C, dtype=torch.bfloat16, seed=87, masked=True).to(DEV)
    out = (torch.empty_like(static.values), torch.empty_like(static.init_slot), torch.empty_like(static.init_mass))
    _launch(nat, static, U, P, K, 2, (0.0, 0.0), False, True, out)  # first call on the device: scratch lookup
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _launch(nat, static, U, P, K, 2, (0.0, 0.0), False, True, out)
    for rep in range(3):
        print(f"no-allocation forward: graph replay {rep}", flush=True)
        fresh = make_case(B=B, H=H, U=U, P=P, T=T, C=C, dtype=torch.bfloat16, seed=88 + rep, masked=True).to(DEV)
        for name in ("w_addr", "r_addr", "values", "gamma", "init_slot", "init_mass", "position_ids", "mask"):
            getattr(static, name).copy_(getattr(fresh, name))
        graph.replay()
        torch.cuda.synchronize()
        want = _launch(nat, fresh, U, P, K, 2, (0.0, 0.0), False, False)
        torch.cuda.synchronize()
        for name, a, b in zip(("y", "slot", "mass"), out, want):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager workspace call"


def test_noalloc_refuses_shapes_beyond_the_scratch():
    """Records of B=8, H=16, T=16384, K=8 need 671 MB, more than the 192 MiB
    scratch: refused with a message before any launch (the pointers are
    never dereferenced)."""
    nat = _nat()
    fake = 0x1000
    B, H, U, P, T, A, C, K = 8, 16, 2, 32, 16384, 1024, 128, 8
    args = [fake, fake, fake, fake, 2, None, 8, fake, fake, fake + 64, fake + 128, fake + 192, fake + 256,
            B, H, U, P, T, A, C, K, K, 0.0, 0.0, 0, 1e-12, None]
    rc = nat.lib().ramnet_ram_attn_forward_noalloc(*args)
    assert rc == nat.RAMNET_EINVAL
    msg = nat.lib().ramnet_last_error().decode()
    assert "scratch" in msg and str(192 << 20) in msg, msg

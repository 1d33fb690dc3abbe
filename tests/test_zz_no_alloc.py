"""``ramnet_ram_attn_forward_noalloc``: the prefill forward with its records
in the library's per-GPU scratch array instead of a caller workspace.

Called through the C ABI and compared with ``ramnet_ram_attn_forward`` (the
same kernels with a caller workspace) on the same inputs: outputs and post
state must be identical bits. Two calls in a row, the second on a smaller
input (the scratch keeps the first call's records, which the second must not
read), then a slot space wide enough for the precomputed-gain form (whose
gain records also live in the scratch), and a shape beyond the scratch, which
is refused on the host before anything is launched.
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


def _run(nat, case, K, E, re_norm, mass_aware, noalloc):
    d = case.to(DEV)
    B, H, U, P, T, C = case.shape
    A = P ** U
    pos = d.position_ids.to(torch.int32).contiguous()
    mask = None if d.mask is None else d.mask.to(torch.uint8).contiguous()
    slot, mass, y = torch.empty_like(d.init_slot), torch.empty_like(d.init_mass), torch.empty_like(d.values)
    code = nat.DTYPE_CODES[d.values.dtype]
    stream = torch.cuda.current_stream().cuda_stream
    args = [d.w_addr.data_ptr(), d.r_addr.data_ptr(), d.values.data_ptr(), d.gamma.data_ptr(), code, nat.ptr(mask), E,
            pos.data_ptr(), d.init_slot.data_ptr(), d.init_mass.data_ptr(), slot.data_ptr(), mass.data_ptr(),
            y.data_ptr(), B, H, U, P, T, A, C, K[0], K[1], re_norm[0], re_norm[1], int(mass_aware), 1e-12]
    if noalloc:
        nat.call("ramnet_ram_attn_forward_noalloc", *args, stream)
    else:
        ws = torch.empty(nat.scan_workspace_bytes(B, H, T, *K), dtype=torch.uint8, device=DEV)
        nat.call("ramnet_ram_attn_forward", *args, ws.data_ptr(), ws.numel(), stream)
    torch.cuda.synchronize()
    return y.cpu(), slot.cpu(), mass.cpu()


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


def test_noalloc_refuses_shapes_beyond_the_scratch():
    """Records of B=8, H=16, T=16384, K=8 need 403 MB, more than the 128 MiB
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
    assert "scratch" in msg and str(128 << 20) in msg, msg

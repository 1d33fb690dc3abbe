"""Build the gfx950 operator library ``libramnet_hip.so`` in-tree with hipcc.

Each HIP translation unit is compiled in parallel into ``_build/`` and the
objects are linked into ``ramnet_ops/_lib/libramnet_hip.so``. Packed-FP32
instruction selection is disabled for device code. The benchmark's LDS
bandwidth probe (``csrc/lds_probe.hip``) is linked into a library of its own,
``ramnet_ops/_lib/libramnet_lds_probe.so``; no operator uses it.

Usage: python ram-net_amd/build_hip.py [--jobs N] [--verbose]
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
BUILD = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "ramnet_ops", "_lib")
LIB = os.path.join(LIB_DIR, "libramnet_hip.so")
PROBE_LIB = os.path.join(LIB_DIR, "libramnet_lds_probe.so")
PROBE_SOURCE = "lds_probe.hip"

SOURCES = ("topk_addr.hip", "segment_forward.hip", "segment_scan_f32.hip", "segment_scan_f16.hip",
           "segment_scan_bf16.hip", "segment_backward.hip", "autoregressive.hip", "capi.hip")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the HIP extension cannot be built")


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-mcode-object-version=5",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", CSRC,
        "-I", INCLUDE,
    ]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops" not in line and line.strip() != "1 warning generated."
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def build(jobs: int | None = None, verbose: bool = False) -> str:
    """Compile every translation unit and link the shared library; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    cc = hipcc()
    objs = []
    cmds = []
    for src in SOURCES + (PROBE_SOURCE,):
        obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        cmds.append([cc, *common_flags(), "-c", os.path.join(CSRC, src), "-o", obj])
    probe_obj = objs.pop()
    jobs = jobs or min(len(cmds), os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        for fut in [pool.submit(_run, c, verbose) for c in cmds]:
            fut.result()
    for lib, lib_objs in ((LIB, objs), (PROBE_LIB, [probe_obj])):
        tmp = lib + ".tmp"
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *lib_objs, "-o", tmp], verbose)
        os.replace(tmp, lib)
    return LIB


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    path = build(args.jobs, args.verbose)
    print(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())

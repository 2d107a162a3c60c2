"""Build libhive_gpu.so (the HIP engine) in-tree for gfx950.

    python -m hive_neuralnet_amd.build

The library is compiled with hipcc straight from csrc/*.hip into
hive_neuralnet_amd/libhive_gpu.so (git-ignored; it travels with the tree).
Flags: no fast-math, no FP contraction (features must be bit-exact with the
reference's IEEE divisions), packed-FP32 instruction selection disabled.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB = os.path.join(PKG, "libhive_gpu.so")
SOURCES = [os.path.join(PKG, "csrc", n) for n in ("hive_engine.hip", "hive_mcts.hip", "hive_fnn.hip", "hive_probe.hip")]
ARCH = os.environ.get("HIVE_GPU_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP engine needs ROCm's hipcc to build")


def build(verbose: bool = False, defines: tuple = (), out: str = LIB) -> str:
    """Compile the library to `out`.  `defines` ("NAME=VALUE") select
    build-time alternatives of the engine, e.g. HW_ANT_GROUP=10 (the lane
    group finishing ant searches after 10 expansions); the package's own
    library is built without any."""
    tmp = out + ".tmp"
    cmd = [hipcc(), *FLAGS, *[f"-D{d}" for d in defines], "-o", tmp, *SOURCES]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed building {out}")
    if verbose:
        sys.stderr.write(res.stderr)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser(description="build the HIP engine library")
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("--define", action="append", default=[], metavar="NAME=VALUE",
                    help="a build-time alternative of the engine (e.g. HW_ANT_GROUP=10)")
    ap.add_argument("--out", default=LIB, help="output path (default: the package's own library)")
    a = ap.parse_args()
    if a.define and os.path.abspath(a.out) == LIB:
        ap.error("a build with --define goes to its own --out path, not the package's library")
    print(build(verbose=a.verbose, defines=tuple(a.define), out=os.path.abspath(a.out)))

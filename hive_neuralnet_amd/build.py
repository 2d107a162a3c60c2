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


def build(verbose: bool = False) -> str:
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *FLAGS, "-o", tmp, *SOURCES]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building libhive_gpu.so")
    if verbose:
        sys.stderr.write(res.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

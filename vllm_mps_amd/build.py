"""Build the HIP sampler library for gfx950, in-tree.

``python -m vllm_mps_amd.build`` compiles ``csrc/mis_sampler.hip`` with hipcc
into ``vllm_mps_amd/_lib/libmis_sampler.so``.  The library exports the C ABI
declared in ``include/mis_sampler.h``.

Flags: no fast-math; hipcc's correctly rounded f32 division (the temperature
division must equal IEEE ``x / T``); packed-FP32 instructions disabled.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
SRC = os.path.join(PKG, "csrc", "mis_sampler.hip")
OUT_DIR = os.path.join(PKG, "_lib")
LIB = os.path.join(OUT_DIR, "libmis_sampler.so")
ARCH = os.environ.get("MIS_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-fast-math", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep each thread's register-resident chunk as separate scalars; promoting
    # it to one wide vector value makes the allocator spill it whole
    "-mllvm", "-disable-promote-alloca-to-vector=true",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the MI355X sampler library cannot be built")


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", os.path.join(ROOT, "include"), "-o", tmp, SRC]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; harmless
    noise = [ln for ln in res.stderr.splitlines() if ln.strip() and "packed-fp32-ops" not in ln]
    if res.returncode != 0:
        sys.stderr.write("\n".join(noise) + "\n")
        raise RuntimeError(f"hipcc failed ({res.returncode})")
    if verbose and noise:
        sys.stderr.write("\n".join(noise) + "\n")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))

"""Build the HIP sampler library for gfx950, in-tree.

``python -m vllm_mps_amd.build`` compiles the translation units under
``csrc/`` with hipcc -- one per logits dtype (``mis_f32.hip``, ``mis_f16.hip``,
``mis_bf16.hip``, built in parallel) and the host-side C ABI (``mis_api.hip``)
-- and links them into ``vllm_mps_amd/_lib/libmis_sampler.so``.  The library
exports the C ABI declared in ``include/mis_sampler.h``.

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
CSRC = os.path.join(PKG, "csrc")
UNITS = ("mis_api.hip", "mis_f32.hip", "mis_f16.hip", "mis_bf16.hip", "mis_rng.hip", "mis_attn.hip", "mis_lmhead.hip")
OUT_DIR = os.path.join(PKG, "_lib")
LIB = os.path.join(OUT_DIR, "libmis_sampler.so")
ARCH = os.environ.get("MIS_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
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


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)


def _finish(proc) -> None:
    out, err = proc.communicate()
    # hipcc's host pass warns that it does not know the packed-fp32 feature; harmless
    noise = [ln for ln in err.splitlines() if ln.strip() and "packed-fp32-ops" not in ln]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}): {' '.join(proc.args)}")


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    cc = hipcc()
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    objs, procs = [], []
    for unit in UNITS:
        obj = os.path.join(OUT_DIR, unit.replace(".hip", ".o"))
        objs.append(obj)
        procs.append(_run([cc, *HIPCC_FLAGS, *inc, "-c", "-o", obj, os.path.join(CSRC, unit)], verbose))
    errors = []
    for p in procs:
        try:
            _finish(p)
        except RuntimeError as e:
            errors.append(str(e))
    if errors:
        raise RuntimeError("; ".join(errors))
    tmp = LIB + ".tmp"
    _finish(_run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose))
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))

"""Build recipe for the CPU emulation of the sampler kernels (test infrastructure).

Compiles the product's translation units (vllm_mps_amd/csrc/mis_*.hip) as
host C++ against the shim in tests/emu/include, together with the fiber
scheduler and driver in tests/emu/emu.cpp, with AddressSanitizer and
array-bounds checks, into tests/emu/_build/emu_driver.  Host-only: no GPU code
is built and nothing here runs on a GPU.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
CSRC = os.path.join(ROOT, "vllm_mps_amd", "csrc")
OUT_DIR = os.path.join(HERE, "_build")
EXE = os.path.join(OUT_DIR, "emu_driver")
EXE_TRACE = os.path.join(OUT_DIR, "emu_driver_trace")
UNITS = ["mis_api.hip", "mis_f32.hip", "mis_f16.hip", "mis_bf16.hip", "mis_rng.hip"]


def clangxx() -> str:
    for c in ("/opt/rocm/llvm/bin/clang++", shutil.which("clang++")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("clang++ not found")


FLAGS = ["-std=c++20", "-O1", "-g", "-fno-omit-frame-pointer", "-ffp-contract=off", "-fno-fast-math",
         "-fsanitize=address", "-fsanitize=bounds", "-fno-sanitize-recover=bounds",
         "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unknown-attributes"]


def sources():
    return [os.path.join(CSRC, u) for u in UNITS] + [os.path.join(HERE, "emu.cpp")]


def up_to_date(exe: str = EXE) -> bool:
    if not os.path.exists(exe):
        return False
    t = os.path.getmtime(exe)
    deps = sources() + [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    deps += [os.path.join(HERE, "include", "hip", "hip_runtime.h"), os.path.join(ROOT, "include", "mis_sampler.h")]
    return all(os.path.getmtime(d) <= t for d in deps)


def build(verbose: bool = False, force: bool = False, trace: bool = False) -> str:
    """trace=True: the kernels' MIS_TRACE phase table as well (emu_driver_trace)."""
    exe = EXE_TRACE if trace else EXE
    if not force and up_to_date(exe):
        return exe
    os.makedirs(OUT_DIR, exist_ok=True)
    cc = clangxx()
    inc = ["-I", os.path.join(HERE, "include"), "-I", os.path.join(ROOT, "include"), "-I", CSRC]
    objs, procs = [], []
    for src in sources():
        obj = os.path.join(OUT_DIR, os.path.basename(src) + (".trace.o" if trace else ".o"))
        objs.append(obj)
        cmd = [cc, *FLAGS, *(["-DMIS_TRACE"] if trace else []), *inc, "-x", "c++", "-c", "-o", obj, src]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append(subprocess.Popen(cmd, stderr=subprocess.PIPE, text=True))
    errs = []
    for p in procs:
        _, err = p.communicate()
        if p.returncode != 0:
            errs.append(err)
    if errs:
        sys.stderr.write("\n".join(errs))
        raise RuntimeError("emulator build failed")
    tmp = exe + ".tmp"
    subprocess.run([cc, *FLAGS, "-o", tmp, *objs], check=True)
    os.replace(tmp, exe)
    return exe


if __name__ == "__main__":
    print(build(verbose=True, force=True))

"""Run a workload through the CPU emulation of the kernels (test infrastructure).

``run(w)`` writes the case file, runs tests/emu/_build/emu_driver and returns
the same dict as ``tests.harness.run_gpu`` (ids, status, probs, keep), so
``oracle.compare.compare`` checks it against the oracle unchanged.
"""
from __future__ import annotations

import os
import struct
import subprocess
import tempfile

import numpy as np

from oracle import compare as C
from tests.emu import build_emu
from vllm_mps_amd import workloads as W

DTYPE_CODE = {"f32": 0, "f16": 1, "bf16": 2}
MAGIC = 0x4D495345


def run(w: W.Workload, debug: bool = True, kinds: int = 7, timeout: float = 600.0, trace: bool = False,
        side: bool = True, noalloc: bool = False) -> dict:
    """trace=True: also returns the MIS_TRACE phase table (``trace`` [B, 32],
    a logical clock: nonzero where a row passed that phase).  side=True:
    with a mis_context (the split schedule), else every launch in one stream.
    noalloc=True: through mis_sample_noalloc (the static scratch; one stream)."""
    exe = build_emu.build(trace=trace)
    B, V = w.shape
    params = np.zeros((B, 4), dtype=np.int32)
    params.view(np.float32)[:, 0] = w.temperature
    params[:, 1] = w.top_k
    params.view(np.float32)[:, 2] = w.top_p
    params.view(np.float32)[:, 3] = w.uniform
    logits = np.ascontiguousarray(w.logits)
    logits = logits.astype(np.float32, copy=False) if w.dtype == "f32" else logits.astype(np.uint16, copy=False)
    with tempfile.TemporaryDirectory() as td:
        cin, cout = os.path.join(td, "case.bin"), os.path.join(td, "out.bin")
        with open(cin, "wb") as f:
            f.write(struct.pack("<iiqqii", MAGIC, DTYPE_CODE[w.dtype], B, V, 1 if debug else 0, kinds))
            f.write(logits.tobytes())
            f.write(params.tobytes())
        env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:detect_stack_use_after_return=0")
        ctr = os.path.join(td, "trace.bin")
        env["EMU_SIDE"] = "1" if side else "0"
        env["EMU_NOALLOC"] = "1" if noalloc else "0"
        if trace:
            env["EMU_TRACE_OUT"] = ctr
        res = subprocess.run([exe, cin, cout], capture_output=True, text=True, timeout=timeout, env=env)
        if res.returncode != 0:
            raise RuntimeError(f"emulator failed ({res.returncode}):\n{res.stderr[-4000:]}")
        raw = open(cout, "rb").read()
        tr = np.fromfile(ctr, dtype=np.uint64).reshape(B, 32) if trace else None
    off = 0
    ids = np.frombuffer(raw, np.int64, B, off); off += 8 * B
    status = np.frombuffer(raw, np.int32, B, off); off += 4 * B
    out = dict(ids=ids.copy(), status=status.copy())
    if tr is not None:
        out["trace"] = tr
    if debug:
        probs = np.frombuffer(raw, np.float32, B * V, off).reshape(B, V); off += 4 * B * V
        Wd = (V + 31) // 32
        keep = np.frombuffer(raw, np.uint32, B * Wd, off).reshape(B, Wd)
        out["probs"] = probs.copy()
        out["keep"] = C.unpack_keep(keep, V)
    return out

"""Python face of the CPU oracle (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module.  It wraps ``mis_oracle.c``, the CPU restatement of
the reference sampler (``model/sampler.py:18-60`` per row, as called from
``engine/llm_engine.py:339-345``).  See the header of ``mis_oracle.c`` for the
exact semantics and the reference line each step follows.

Logits cross this boundary as raw numpy arrays: ``float32`` for fp32, and the
16-bit patterns as ``uint16`` for fp16 and bf16 (numpy has no bf16).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import build as _build

DTYPE_CODES = {"f32": 0, "f16": 1, "bf16": 2}

_lib = None


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_build.LIB):
        _build.build_oracle()
    lib = ctypes.CDLL(_build.LIB)
    p = ctypes.c_void_p
    i64 = ctypes.c_int64
    lib.orc_sample_rows.argtypes = [ctypes.c_int, i64, i64, i64, p, p, p, p, p, p, p, p, p, p, p]
    lib.orc_sample_rows.restype = ctypes.c_int
    lib.orc_scale_array.argtypes = [ctypes.c_int, i64, p, ctypes.c_float, p]
    lib.orc_round_array.argtypes = [ctypes.c_int, i64, p, p]
    lib.orc_f32_to_f16.argtypes = [ctypes.c_float]
    lib.orc_f32_to_f16.restype = ctypes.c_uint16
    lib.orc_f32_to_bf16.argtypes = [ctypes.c_float]
    lib.orc_f32_to_bf16.restype = ctypes.c_uint16
    lib.orc_philox4x32_10.argtypes = [p, p, p]
    lib.orc_uniforms.argtypes = [i64, p, p, p, p]
    _lib = lib
    return lib


PARAMS_DTYPE = np.dtype([("temperature", "<f4"), ("top_k", "<i4"), ("top_p", "<f4"), ("uniform", "<f4")])


def make_params(temperature, top_k, top_p, uniform) -> np.ndarray:
    """Pack per-row parameters into the 16-byte record the C code reads."""
    t = np.atleast_1d(np.asarray(temperature, dtype=np.float32))
    n = t.shape[0]
    out = np.zeros(n, dtype=PARAMS_DTYPE)
    out["temperature"] = t
    out["top_k"] = np.broadcast_to(np.asarray(top_k, dtype=np.int32), (n,))
    out["top_p"] = np.broadcast_to(np.asarray(top_p, dtype=np.float32), (n,))
    out["uniform"] = np.broadcast_to(np.asarray(uniform, dtype=np.float32), (n,))
    return out


def _raw(logits: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "f32":
        assert logits.dtype == np.float32
    elif dtype == "f16":
        logits = logits.view(np.uint16) if logits.dtype == np.float16 else logits
        assert logits.dtype == np.uint16
    else:
        assert logits.dtype == np.uint16, "bf16 logits travel as uint16 bit patterns"
    return np.ascontiguousarray(logits)


def sample_rows(logits: np.ndarray, dtype: str, params: np.ndarray, want_probs=False, want_keep=False):
    """Run the oracle over a [B, V] batch.  Returns a dict of numpy arrays:
    ids, status, topp_margin, draw_margin, cut_value, cut_index, n_kept and,
    on request, probs [B, V] float32 and keep [B, V] bool."""
    lib = _load()
    raw = _raw(logits, dtype)
    B, V = raw.shape
    assert params.dtype == PARAMS_DTYPE and params.shape == (B,)
    params = np.ascontiguousarray(params)
    ids = np.empty(B, np.int64)
    status = np.empty(B, np.int32)
    tm = np.empty(B, np.float64)
    dm = np.empty(B, np.float64)
    cv = np.empty(B, np.float32)
    ci = np.empty(B, np.int64)
    nk = np.empty(B, np.int64)
    probs = np.empty((B, V), np.float32) if want_probs else None
    keep = np.empty((B, V), np.uint8) if want_keep else None
    ptr = lambda a: None if a is None else a.ctypes.data_as(ctypes.c_void_p)
    rc = lib.orc_sample_rows(DTYPE_CODES[dtype], B, V, V, ptr(raw), ptr(params), ptr(ids), ptr(status),
                             ptr(probs), ptr(keep), ptr(tm), ptr(dm), ptr(cv), ptr(ci), ptr(nk))
    if rc != 0:
        raise RuntimeError(f"oracle failed: {rc}")
    out = dict(ids=ids, status=status, topp_margin=tm, draw_margin=dm, cut_value=cv,
               cut_index=ci, n_kept=nk)
    if want_probs:
        out["probs"] = probs
    if want_keep:
        out["keep"] = keep.astype(bool)
    return out


def scale(x: np.ndarray, dtype: str, T: float) -> np.ndarray:
    """y = dtype(f32(x) / f32(T)) as float32 (sampler.py:37)."""
    lib = _load()
    raw = _raw(np.ascontiguousarray(x).reshape(-1), dtype)
    y = np.empty(raw.shape[0], np.float32)
    lib.orc_scale_array(DTYPE_CODES[dtype], raw.shape[0], raw.ctypes.data_as(ctypes.c_void_p),
                        ctypes.c_float(T), y.ctypes.data_as(ctypes.c_void_p))
    return y


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to the dtype (RNE), returned as float32."""
    lib = _load()
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    y = np.empty_like(x)
    lib.orc_round_array(DTYPE_CODES[dtype], x.shape[0], x.ctypes.data_as(ctypes.c_void_p),
                        y.ctypes.data_as(ctypes.c_void_p))
    return y


def philox4x32_10(counter, key) -> np.ndarray:
    """Philox4x32-10 of one 128-bit counter (4 words) under a 64-bit key (2 words)."""
    c = np.ascontiguousarray(counter, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    _load().orc_philox4x32_10(c.ctypes.data, k.ctypes.data, out.ctypes.data)
    return out


def uniforms(seed, request, step) -> np.ndarray:
    """Per-request uniforms of the device generator (broadcast uint64 arrays)."""
    s, r, t = (np.ascontiguousarray(a, dtype=np.uint64) for a in np.broadcast_arrays(seed, request, step))
    out = np.zeros(s.shape, dtype=np.float32)
    _load().orc_uniforms(s.size, s.ctypes.data, r.ctypes.data, t.ctypes.data, out.ctypes.data)
    return out

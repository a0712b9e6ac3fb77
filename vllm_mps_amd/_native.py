"""ctypes binding of the C ABI in ``include/mis_sampler.h``.

The product path has no CPU or eager fallback: if ``libmis_sampler.so`` is
missing or does not load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

from . import build as _build

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
ROW_OK, ROW_BAD_PARAM, ROW_INVALID, ROW_UNSUPPORTED, ROW_INTERNAL = 0, 1, 2, 3, 4
ABI_VERSION = 8
SCRATCH_BYTES = 128 << 20  # MIS_SCRATCH_BYTES: the static scratch of mis_sample_noalloc
ERR_SCRATCH = 5  # MIS_ERR_SCRATCH
KIND_TOPP32 = 1  # MIS_KIND_TOPP32
KIND_OTHER = 2   # MIS_KIND_OTHER
KIND_GENERIC = 4  # MIS_KIND_GENERIC
KIND_ALL = 7     # MIS_KIND_ALL

EXPORTED = ("mis_workspace_bytes", "mis_workspace_init", "mis_sample", "mis_sample_profiled", "mis_sample_ex",
            "mis_sample_noalloc", "mis_fill_uniforms", "mis_context_create",
            "mis_paged_attention_workspace_bytes", "mis_paged_attention", "mis_gather_kv",
            "mis_lm_head_greedy_workspace_bytes", "mis_lm_head_greedy", "mis_lm_head_sample", "mis_context_destroy", "mis_strerror", "mis_last_hip_error", "mis_abi_version")

_lib = None


class MisError(RuntimeError):
    pass


def lib_path() -> str:
    return os.environ.get("MIS_SAMPLER_LIB", _build.LIB)


def load():
    """Load (once) and return the native library; raises MisError when absent."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not os.path.exists(path):
        raise MisError(f"MI355X sampler library not built: {path} is missing "
                       "(run `python -m vllm_mps_amd.build`); there is no CPU fallback")
    lib = ctypes.CDLL(path)
    i64, vp = ctypes.c_int64, ctypes.c_void_p
    lib.mis_workspace_bytes.argtypes = [i64, i64, ctypes.c_int]
    lib.mis_workspace_bytes.restype = ctypes.c_size_t
    lib.mis_workspace_init.argtypes = [vp, ctypes.c_size_t, vp]
    lib.mis_workspace_init.restype = ctypes.c_int
    lib.mis_sample.argtypes = [vp, ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, vp, ctypes.c_size_t, vp]
    lib.mis_sample.restype = ctypes.c_int
    lib.mis_sample_profiled.argtypes = [vp, ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, vp, ctypes.c_size_t, vp,
                                        ctypes.POINTER(vp)]
    lib.mis_sample_profiled.restype = ctypes.c_int
    lib.mis_sample_ex.argtypes = [vp, ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, vp, ctypes.c_size_t, vp,
                                  ctypes.c_uint, vp, vp]
    lib.mis_sample_ex.restype = ctypes.c_int
    lib.mis_sample_noalloc.argtypes = [vp, ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, vp, ctypes.c_uint]
    lib.mis_sample_noalloc.restype = ctypes.c_int
    lib.mis_fill_uniforms.argtypes = [vp, vp, i64, vp]
    lib.mis_fill_uniforms.restype = ctypes.c_int
    ci = ctypes.c_int
    lib.mis_paged_attention_workspace_bytes.argtypes = [i64, ci, ci, ci, ci]
    lib.mis_paged_attention_workspace_bytes.restype = ctypes.c_size_t
    lib.mis_paged_attention.argtypes = [vp, i64, ci, ci, ci, i64, i64, vp, vp, vp, vp, ci, vp, vp, i64, ci, vp, vp,
                                        ctypes.c_size_t, vp]
    lib.mis_paged_attention.restype = ci
    lib.mis_gather_kv.argtypes = [vp, i64, ci, ci, ci, i64, i64, vp, ci, vp, i64, ci, vp, vp, vp]
    lib.mis_gather_kv.restype = ci
    lib.mis_lm_head_greedy_workspace_bytes.argtypes = [i64, i64]
    lib.mis_lm_head_greedy_workspace_bytes.restype = ctypes.c_size_t
    lib.mis_lm_head_greedy.argtypes = [vp, i64, vp, i64, i64, i64, i64, ci, vp, vp, ctypes.c_size_t, vp]
    lib.mis_lm_head_greedy.restype = ci
    lib.mis_lm_head_sample.argtypes = [vp, i64, vp, i64, i64, i64, i64, ci, vp, vp, vp, vp, ctypes.c_size_t, vp]
    lib.mis_lm_head_sample.restype = ci
    lib.mis_context_create.argtypes = [ctypes.POINTER(vp)]
    lib.mis_context_create.restype = ctypes.c_int
    lib.mis_context_destroy.argtypes = [vp]
    lib.mis_context_destroy.restype = ctypes.c_int
    lib.mis_strerror.argtypes = [ctypes.c_int]
    lib.mis_strerror.restype = ctypes.c_char_p
    lib.mis_last_hip_error.restype = ctypes.c_int
    lib.mis_abi_version.restype = ctypes.c_int
    if lib.mis_abi_version() != ABI_VERSION:
        raise MisError(f"ABI mismatch: library {lib.mis_abi_version()} != {ABI_VERSION}")
    _lib = lib
    return lib


def workspace_bytes(B: int, V: int, dtype: int) -> int:
    return int(load().mis_workspace_bytes(B, V, dtype))


def workspace_init(ws_ptr: int, ws_bytes: int, stream: int) -> None:
    """Clear a new workspace's control words (once, before its first use)."""
    lib = load()
    rc = lib.mis_workspace_init(ws_ptr, ws_bytes, stream)
    if rc != 0:
        raise MisError(f"mis_workspace_init failed: {lib.mis_strerror(rc).decode()}")


def fill_uniforms(params_ptr: int, rng_ptr: int, B: int, stream: int) -> None:
    """mis_fill_uniforms: params[r].uniform from the device generator state
    rng[r] = (seed, request, step), 24 bytes a row."""
    lib = load()
    rc = lib.mis_fill_uniforms(params_ptr, rng_ptr, B, stream)
    if rc != 0:
        msg = lib.mis_strerror(rc).decode()
        if rc == 3:
            msg += f" (hipError {lib.mis_last_hip_error()})"
        raise MisError(f"mis_fill_uniforms failed: {msg}")


class Context:
    """A mis_context: a side stream and its fork / join events on the device
    current at creation (mis_context_create); destroyed with the object."""

    def __init__(self) -> None:
        self._lib = load()
        h = ctypes.c_void_p()
        rc = self._lib.mis_context_create(ctypes.byref(h))
        if rc != 0:
            raise MisError(f"mis_context_create failed: {self._lib.mis_strerror(rc).decode()} "
                           f"(hipError {self._lib.mis_last_hip_error()})")
        self.handle = h.value

    def close(self) -> None:
        if getattr(self, "handle", None):
            self._lib.mis_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def sample(logits_ptr: int, dtype: int, B: int, V: int, row_stride: int, params_ptr: int, ids_ptr: int,
           status_ptr: int | None, probs_ptr: int | None, keep_ptr: int | None, ws_ptr: int, ws_bytes: int,
           stream: int, events: tuple | None = None, kinds: int | None = None, context: Context | None = None) -> None:
    """events: None, or three handles (mis_sample_profiled), or four with
    kinds (mis_sample_ex: the fourth closes the side stream's chunk pass).
    context: a Context for mis_sample_ex's split schedule (needs kinds)."""
    lib = load()
    if context is not None and kinds is None:
        kinds = KIND_ALL
    if kinds is not None:
        if events is not None and len(events) != 4:
            raise ValueError("mis_sample_ex takes four events")
        ev = None if events is None else (ctypes.c_void_p * 4)(*events)
        rc = lib.mis_sample_ex(logits_ptr, dtype, B, V, row_stride, params_ptr, ids_ptr, status_ptr, probs_ptr,
                               keep_ptr, ws_ptr, ws_bytes, stream, kinds, ev,
                               None if context is None else context.handle)
    elif events is None:
        rc = lib.mis_sample(logits_ptr, dtype, B, V, row_stride, params_ptr, ids_ptr, status_ptr, probs_ptr,
                            keep_ptr, ws_ptr, ws_bytes, stream)
    else:
        ev = (ctypes.c_void_p * 3)(*events)
        rc = lib.mis_sample_profiled(logits_ptr, dtype, B, V, row_stride, params_ptr, ids_ptr, status_ptr,
                                     probs_ptr, keep_ptr, ws_ptr, ws_bytes, stream, ev)
    if rc != 0:
        msg = lib.mis_strerror(rc).decode()
        if rc == 3:
            msg += f" (hipError {lib.mis_last_hip_error()})"
        raise MisError(f"mis_sample failed: {msg}")


def sample_noalloc(logits_ptr: int, dtype: int, B: int, V: int, row_stride: int, params_ptr: int, ids_ptr: int,
                   status_ptr: int | None, probs_ptr: int | None, keep_ptr: int | None, stream: int,
                   kinds: int = KIND_ALL) -> None:
    """mis_sample_noalloc: no workspace; the library's static per-device
    scratch (SCRATCH_BYTES) serves instead.  Calls that overlap on one device
    race on it."""
    lib = load()
    rc = lib.mis_sample_noalloc(logits_ptr, dtype, B, V, row_stride, params_ptr, ids_ptr, status_ptr, probs_ptr,
                                keep_ptr, stream, kinds)
    if rc != 0:
        msg = lib.mis_strerror(rc).decode()
        if rc == 3:
            msg += f" (hipError {lib.mis_last_hip_error()})"
        raise MisError(f"mis_sample_noalloc failed: {msg}")

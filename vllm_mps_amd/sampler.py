"""Drop-in ``Sampler`` for the decode step, backed by the MI355X HIP kernels.

Mirrors the reference's ``Sampler`` (``model/sampler.py:11-79``):

* ``Sampler()`` -- no-argument constructor, as the engine builds it
  (``engine/llm_engine.py:108,180``).
* ``sample(logits[V], params) -> int`` (``model/sampler.py:18``).
* ``sample_batch(logits[B, V], params) -> list[int]`` (``model/sampler.py:62``).

and adds the batched entry point the engine's per-row loop
(``engine/llm_engine.py:339-345``) collapses into:

* ``sample_rows(logits[B, V], params_per_row, uniforms=None, rng=None) ->
  int64[B]`` on the device, one launch sequence and no host synchronisation.

Differences from the reference, all contract decisions:
* the draw is an inverse CDF in vocabulary order from one uniform per row
  instead of ``torch.multinomial``; uniforms come from ``torch.rand`` on the
  device (``generator`` selects the stream) unless the caller passes them or
  asks for the per-request device generator (``rng``);
* top-p ties at the cut keep the lowest indices first (stable order);
* fp32 top-p masses are exact softmax masses, not torch's float softmax.

There is no CPU path: logits must live on a ROCm device and the native
library must be built, otherwise the calls raise.
"""
from __future__ import annotations

from typing import Sequence

import numpy as np
import torch

from . import _native
from .sampling_params import SamplingParams

_DTYPES = {torch.float32: _native.DTYPE_F32, torch.float16: _native.DTYPE_F16, torch.bfloat16: _native.DTYPE_BF16}
_ONE_BELOW = float(np.nextafter(np.float32(1.0), np.float32(0.0)))


def dtype_code(dtype: torch.dtype) -> int:
    if dtype not in _DTYPES:
        raise TypeError(f"logits dtype {dtype} not supported (float32, float16, bfloat16)")
    return _DTYPES[dtype]


def host_row_params(params: Sequence[SamplingParams], dtype: torch.dtype) -> np.ndarray:
    """[B, 3] (temperature f32, top_k i32, top_p f32) packed as int32 words.

    Python floats become the f32 values torch would use: the temperature is
    divided as ``f32(x) / f32(T)`` and ``top_p`` is compared after a cast to
    the logits dtype (probed on torch 2.10).  A top_p below 1.0 whose f32
    rounding is 1.0 stays active for 16-bit logits (threshold RN16 = 1.0)
    and is a no-op for fp32 logits (exact masses never reach 1.0 early).
    """
    B = len(params)
    out = np.zeros((B, 3), dtype=np.int32)
    f = out.view(np.float32)
    for i, sp in enumerate(params):
        t = float(sp.temperature)
        t32 = np.float32(t)
        if t > 0.0 and t32 == 0.0:
            # torch divides by f32(T) = 0: inf / NaN logits, and multinomial
            # raises; NaN selects that row status (invalid distribution)
            t32 = np.float32(np.nan)
        f[i, 0] = t32
        out[i, 1] = int(min(max(int(sp.top_k), 0), 2**31 - 1)) if sp.top_k >= 0 else int(sp.top_k)
        p = float(sp.top_p)
        p32 = np.float32(p)
        if p < 1.0 and p32 == np.float32(1.0) and dtype != torch.float32:
            p32 = np.float32(_ONE_BELOW)
        f[i, 2] = p32
    return out


def rng_rows(B: int, seed, requests, steps) -> np.ndarray:
    """[B, 3] uint64 ``mis_rng_row`` records (seed, request, step); each
    argument is a scalar or a length-B sequence of non-negative integers
    below 2^64."""
    out = np.zeros((B, 3), dtype=np.uint64)
    for j, v in enumerate((seed, requests, steps)):
        a = np.asarray(v, dtype=object).reshape(-1) if not np.isscalar(v) else np.array([v], dtype=object)
        if a.size not in (1, B):
            raise ValueError(f"generator state needs 1 or {B} values, got {a.size}")
        for x in a:
            if not 0 <= int(x) < 1 << 64:
                raise ValueError(f"generator state value {x} outside [0, 2^64)")
        out[:, j] = np.array([int(x) for x in a], dtype=np.uint64)
    return out


KIND_TOPP32 = _native.KIND_TOPP32
KIND_OTHER = _native.KIND_OTHER
KIND_GENERIC = _native.KIND_GENERIC


def row_kinds(temperature, top_k, top_p, V: int, dtype: torch.dtype) -> int:
    """Row-kind hint for ``mis_sample_ex`` from host-side per-row parameters
    (sequences or arrays of floats/ints): which kinds the batch holds.
    * TOPP32: fp32 logits with 0 < T, top-k off (0 or >= V) and top_p < 1;
    * OTHER: every other row;
    * GENERIC: among the others, rows the generic row pass serves (0 < T and
      1024 < top_k < V, or 16-bit logits with top-k off and top_p < 1).
    Only a performance hint: the results do not depend on it."""
    t = np.asarray(temperature, dtype=np.float64).reshape(-1)
    k = np.asarray(top_k, dtype=np.int64).reshape(-1)
    p = np.asarray(top_p, dtype=np.float64).reshape(-1)
    if t.size == 0:
        return 0
    stoch = ~(t == 0)  # NaN temperatures are rejected rows, not greedy
    k_off = (k <= 0) | (k >= V)
    p_on = (np.float32(1.0) > p.astype(np.float32)) & (p > 0)
    if dtype == torch.float32:
        topp = stoch & k_off & p_on
    else:
        topp = np.zeros_like(stoch)
    generic = stoch & ((k > 1024) & (k < V) | (dtype != torch.float32) & k_off & p_on)
    kinds = 0
    if topp.any():
        kinds |= KIND_TOPP32
    if (~topp).any():
        kinds |= KIND_OTHER
    if generic.any():
        kinds |= KIND_GENERIC
    return kinds


def pack_params(temperature: torch.Tensor, top_k: torch.Tensor, top_p: torch.Tensor, uniform: torch.Tensor) -> torch.Tensor:
    """Device [B, 4] int32 buffer laid out as ``mis_row_params``."""
    return torch.stack([temperature.to(torch.float32).view(torch.int32), top_k.to(torch.int32),
                        top_p.to(torch.float32).view(torch.int32), uniform.to(torch.float32).view(torch.int32)],
                       dim=1).contiguous()


class Sampler:
    """Samples the next token of every row on the GPU."""

    def __init__(self, generator: torch.Generator | None = None) -> None:
        self.generator = generator
        self._workspace: dict[int, torch.Tensor] = {}
        self._context: dict[int, _native.Context] = {}

    # -- workspace -------------------------------------------------------
    def workspace(self, device: torch.device, B: int, V: int, code: int) -> torch.Tensor:
        need = _native.workspace_bytes(B, V, code)
        idx = device.index if device.index is not None else torch.cuda.current_device()
        ws = self._workspace.get(idx)
        if ws is None or ws.numel() < need:
            ws = torch.empty(need, dtype=torch.uint8, device=device)
            # the kernels keep no state in it between calls; the init call is
            # part of the ABI contract and cheap
            _native.workspace_init(ws.data_ptr(), ws.numel(), torch.cuda.current_stream(device).cuda_stream)
            self._workspace[idx] = ws
        return ws

    def context(self, device: torch.device) -> _native.Context:
        """This sampler's side stream on `device` (made once, kept with the
        sampler, as the engine keeps one Sampler: engine/llm_engine.py:108)."""
        idx = device.index if device.index is not None else torch.cuda.current_device()
        ctx = self._context.get(idx)
        if ctx is None:
            with torch.cuda.device(idx):
                ctx = _native.Context()
            self._context[idx] = ctx
        return ctx

    # -- batched device entry point ---------------------------------------
    def sample_packed(self, logits: torch.Tensor, packed: torch.Tensor, *, out: torch.Tensor | None = None,
                      status_out: torch.Tensor | None = None, probs_out: torch.Tensor | None = None,
                      keep_out: torch.Tensor | None = None, events=None, kinds: int | None = None) -> torch.Tensor:
        """One launch sequence over ``logits[B, V]`` with a device ``packed``
        [B, 4] int32 parameter buffer (see ``pack_params``).  ``events``: recorded
        ``torch.cuda.Event`` objects timing the chunk pass and the row pass:
        three without ``kinds`` (``mis_sample_profiled``), four with it
        (``mis_sample_ex``: the fourth closes the side stream's chunk pass).  ``kinds``: the row-kind hint
        (``row_kinds``), None for "any"."""
        if logits.dim() != 2:
            raise ValueError("logits must be [B, V]")
        if logits.device.type != "cuda":
            raise _native.MisError("the MI355X sampler needs logits on a ROCm device; there is no CPU path")
        code = dtype_code(logits.dtype)
        if logits.stride(1) != 1:
            logits = logits.contiguous()
        B, V = logits.shape
        dev = logits.device
        if out is None:
            out = torch.empty(B, dtype=torch.int64, device=dev)
        for t, dt, shape in ((packed, torch.int32, (B, 4)), (out, torch.int64, (B,)),
                             (status_out, torch.int32, (B,)), (probs_out, torch.float32, (B, V)),
                             (keep_out, torch.int32, (B, (V + 31) // 32))):
            if t is not None and (t.dtype != dt or tuple(t.shape) != shape or not t.is_contiguous() or t.device != dev):
                raise ValueError(f"buffer must be a contiguous {dt} {shape} tensor on {dev}")
        ws = self.workspace(dev, B, V, code)
        stream = torch.cuda.current_stream(dev).cuda_stream
        ptr = lambda t: None if t is None else t.data_ptr()
        evs = None if events is None else tuple(int(e.cuda_event) for e in events)
        ctx = self.context(dev) if kinds is not None else None
        _native.sample(logits.data_ptr(), code, B, V, logits.stride(0), packed.data_ptr(), out.data_ptr(),
                       ptr(status_out), ptr(probs_out), ptr(keep_out), ws.data_ptr(), ws.numel(), stream, evs,
                       kinds=kinds, context=ctx)
        return out

    def sample_rows(self, logits: torch.Tensor, params: Sequence[SamplingParams],
                    uniforms: torch.Tensor | None = None, rng=None, **buffers) -> torch.Tensor:
        """Per-row params, device int64[B] token ids (-1 where a row is invalid).

        The draw's uniforms: ``uniforms`` when given; else, with ``rng =
        (seed, requests, steps)`` (scalars or length-B integer sequences),
        the per-request device generator (``mis_fill_uniforms``: a row's
        uniform depends only on its seed, request and step); else
        ``torch.rand`` with this sampler's ``generator``."""
        B = logits.shape[0]
        if len(params) != B:
            raise ValueError(f"{len(params)} SamplingParams for {B} rows")
        dev = logits.device
        if dev.type != "cuda":
            raise _native.MisError("the MI355X sampler needs logits on a ROCm device; there is no CPU path")
        hp = host_row_params(params, logits.dtype)
        host = torch.from_numpy(hp)
        hf = hp.view(np.float32)
        buffers.setdefault("kinds", row_kinds(hf[:, 0], hp[:, 1], hf[:, 2], logits.shape[1], logits.dtype))
        if uniforms is None and rng is None:
            uniforms = torch.rand(B, device=dev, dtype=torch.float32, generator=self.generator)
        packed = torch.empty((B, 4), dtype=torch.int32, device=dev)
        # staged through pinned host memory: the copy is queued on the stream
        # and the host does not wait for the device
        packed[:, :3].copy_(host.pin_memory(), non_blocking=True)
        if uniforms is not None:
            packed[:, 3].copy_(uniforms.to(device=dev, dtype=torch.float32).view(torch.int32))
        elif B > 0:
            state = torch.from_numpy(rng_rows(B, *rng).view(np.int64)).pin_memory()
            dstate = torch.empty((B, 3), dtype=torch.int64, device=dev)
            dstate.copy_(state, non_blocking=True)
            _native.fill_uniforms(packed.data_ptr(), dstate.data_ptr(), B, torch.cuda.current_stream(dev).cuda_stream)
        return self.sample_packed(logits, packed, **buffers)

    # -- reference call surface -------------------------------------------
    def _checked(self, ids: torch.Tensor, status: torch.Tensor) -> list[int]:
        """Host ints, raising as the reference does for a row it rejects:
        ValueError for invalid parameters (core/sequence.py:41-61),
        RuntimeError for an invalid distribution (torch.multinomial,
        model/sampler.py:59)."""
        st = status.tolist()
        for s in st:
            if s == _native.ROW_BAD_PARAM:
                raise ValueError("invalid sampling parameters")
            if s == _native.ROW_INVALID:
                raise RuntimeError("invalid probability distribution (NaN/inf logits or nothing left to sample)")
            if s == _native.ROW_UNSUPPORTED:
                raise NotImplementedError("row not served by the sampler library (status 3)")
            if s != _native.ROW_OK:
                raise _native.MisError(f"sampler row status {s}")
        return ids.tolist()

    def sample(self, logits: torch.Tensor, sampling_params: SamplingParams) -> int:
        """Sample one token from ``logits[V]`` (model/sampler.py:18)."""
        if logits.dim() != 1:
            raise ValueError("logits must be [V]")
        status = torch.empty(1, dtype=torch.int32, device=logits.device)
        ids = self.sample_rows(logits.unsqueeze(0), [sampling_params], status_out=status)
        return self._checked(ids, status)[0]

    def sample_batch(self, logits_batch: torch.Tensor, sampling_params: SamplingParams) -> list[int]:
        """One token per row with shared params (model/sampler.py:62)."""
        B = logits_batch.shape[0]
        status = torch.empty(B, dtype=torch.int32, device=logits_batch.device)
        ids = self.sample_rows(logits_batch, [sampling_params] * B, status_out=status)
        return self._checked(ids, status)

"""The lm_head GEMM fused with the greedy / temperature sampler on the MI355X (HIP kernel
``mis_lmhead.hip``, C ABI ``include/mis_lmhead.h``).

Replaces, for greedy rows, the producer of the decode step's logits (the
model's lm_head, ``models/llama_adapter.py:198-207``) together with the
sampler's greedy branch (``torch.argmax(logits)``, ``model/sampler.py:32-34``):
the logits are never written to HBM.  ``lm_head_greedy(hidden, weight)``
returns ``argmax(dtype(hidden @ weight.T), dim=-1)`` with the sum in fp32 and
one rounding to the model dtype, ties to the lowest index, NaN first.
``lm_head_sample(hidden, weight, temperature, rng)`` also serves temperature-only
rows (``model/sampler.py:37, :57-59`` with top-k 0 and top-p 1, the default
parameters): the Gumbel-max draw argmax(dtype(logit / T) + g) from softmax,
with g from a per-request counter-based generator.  There is no CPU path.
"""
from __future__ import annotations

import torch

from . import _native

_DT = {torch.float16: 1, torch.bfloat16: 2}
_workspace: dict[int, torch.Tensor] = {}


def lm_head_greedy(hidden: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """hidden [B, H] and weight [V, H] (fp16 or bf16, the same dtype, on a ROCm
    device; rows contiguous) -> int64 ids [B] on the device."""
    if hidden.device.type != "cuda" or weight.device != hidden.device:
        raise _native.MisError("lm_head_greedy needs hidden and weight on one ROCm device; there is no CPU path")
    if hidden.dtype not in _DT or weight.dtype != hidden.dtype:
        raise ValueError("hidden and weight must both be float16 or both bfloat16")
    if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError("hidden must be [B, H] and weight [V, H]")
    if hidden.stride(1) != 1 or weight.stride(1) != 1:
        raise ValueError("hidden and weight rows must be contiguous")
    lib = _native.load()
    B, H = hidden.shape
    V = weight.shape[0]
    dev = hidden.device
    ids = torch.empty(B, dtype=torch.int64, device=dev)
    need = int(lib.mis_lm_head_greedy_workspace_bytes(B, V))
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _workspace.get(idx)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        _workspace[idx] = ws
    rc = lib.mis_lm_head_greedy(hidden.data_ptr(), hidden.stride(0), weight.data_ptr(), weight.stride(0), B, H, V,
                                _DT[hidden.dtype], ids.data_ptr(), ws.data_ptr(), ws.numel(),
                                torch.cuda.current_stream(dev).cuda_stream)
    _check(rc, "mis_lm_head_greedy")
    return ids


def _check(rc: int, what: str) -> None:
    if rc != 0:
        names = {1: "invalid argument", 2: "workspace", 3: "HIP launch failed", 4: "unsupported shape"}
        raise _native.MisError(f"{what} failed: {names.get(rc, rc)}")


def lm_head_sample(hidden: torch.Tensor, weight: torch.Tensor, temperature, rng) -> torch.Tensor:
    """Greedy and temperature-only rows in one fused call (``mis_lm_head_sample``):
    temperature [B] (0 = greedy), rng = (seed, requests [B], steps [B]) keying
    each row's Gumbel noise (a request's token depends only on its logits and
    (seed, request, step)), or those records already on the device
    (``rng_rows``).  int64 ids [B] on the device; -1 for an invalid row.
    Top-k / top-p rows need the unfused path."""
    if hidden.device.type != "cuda" or weight.device != hidden.device:
        raise _native.MisError("lm_head_sample needs hidden and weight on one ROCm device; there is no CPU path")
    if hidden.dtype not in _DT or weight.dtype != hidden.dtype:
        raise ValueError("hidden and weight must both be float16 or both bfloat16")
    if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError("hidden must be [B, H] and weight [V, H]")
    if hidden.stride(1) != 1 or weight.stride(1) != 1:
        raise ValueError("hidden and weight rows must be contiguous")
    lib = _native.load()
    B, H = hidden.shape
    V = weight.shape[0]
    dev = hidden.device
    t = torch.as_tensor(temperature, dtype=torch.float32).to(dev).reshape(-1).contiguous()
    if isinstance(rng, torch.Tensor):
        rows = rng                             # already [B, 3] int64 (mis_rng_row) on the device
    else:
        rows = rng_rows(rng, B, dev)
    if t.numel() != B or rows.shape != (B, 3) or rows.dtype != torch.int64 or rows.device != dev \
            or not rows.is_contiguous():
        raise ValueError("temperature needs one entry per row and rng (seed, requests, steps) one per row")
    ids = torch.empty(B, dtype=torch.int64, device=dev)
    need = int(lib.mis_lm_head_greedy_workspace_bytes(B, V))
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _workspace.get(idx)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        _workspace[idx] = ws
    rc = lib.mis_lm_head_sample(hidden.data_ptr(), hidden.stride(0), weight.data_ptr(), weight.stride(0), B, H, V,
                                _DT[hidden.dtype], t.data_ptr(), rows.data_ptr(), ids.data_ptr(), ws.data_ptr(),
                                ws.numel(), torch.cuda.current_stream(dev).cuda_stream)
    _check(rc, "mis_lm_head_sample")
    return ids


def rng_rows(rng, B: int, device) -> torch.Tensor:
    """(seed, requests [B], steps [B]) -> the [B, 3] int64 mis_rng_row records on `device`;
    build them once per step and pass the tensor to lm_head_sample to keep the
    host-to-device copy out of the call."""
    seed, requests, steps = rng
    req = torch.as_tensor(requests, dtype=torch.int64).reshape(-1)
    stp = torch.as_tensor(steps, dtype=torch.int64).reshape(-1)
    if req.numel() != B or stp.numel() != B:
        raise ValueError("requests and steps need one entry per row")
    rows = torch.stack([torch.full((B,), _i64(seed), dtype=torch.int64), req, stp], dim=1)
    return rows.contiguous().to(device)


def _i64(x: int) -> int:
    """A 64-bit unsigned value as the int64 with the same bits."""
    x = int(x) & 0xFFFFFFFFFFFFFFFF
    return x - (1 << 64) if x >= 1 << 63 else x

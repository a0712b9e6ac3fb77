"""The lm_head GEMM fused with the greedy sampler on the MI355X (HIP kernel
``mis_lmhead.hip``, C ABI ``include/mis_lmhead.h``).

Replaces, for greedy rows, the producer of the decode step's logits (the
model's lm_head, ``models/llama_adapter.py:198-207``) together with the
sampler's greedy branch (``torch.argmax(logits)``, ``model/sampler.py:32-34``):
the logits are never written to HBM.  ``lm_head_greedy(hidden, weight)``
returns ``argmax(dtype(hidden @ weight.T), dim=-1)`` with the sum in fp32 and
one rounding to the model dtype, ties to the lowest index, NaN first.  There
is no CPU path.
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
    if rc != 0:
        names = {1: "invalid argument", 2: "workspace", 3: "HIP launch failed", 4: "unsupported shape"}
        raise _native.MisError(f"mis_lm_head_greedy failed: {names.get(rc, rc)}")
    return ids

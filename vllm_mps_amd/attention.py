"""Decode-step paged attention on the MI355X (HIP kernel ``mis_attn.hip``).

Drop-in for the reference's Metal entry points (``kernels/__init__.py``):

* ``fused_attention_fast`` = ``fused_attention_metal_fast`` (``:320-368``):
  writes the step's new K / V into the block pool, then attention of every
  query head over its sequence's blocks, one call for the batch;
* ``fused_attention`` = ``fused_attention_metal`` (``:371-405``): the same
  from Python lists of block tables and write positions;
* ``gather_kv`` = ``gather_kv_metal`` (``:279-311``): the pool gathered into
  dense [B, max_seq_len, n_kv_heads, d_k] K and V.

The pool is the reference's [num_blocks, 2, block_size, n_kv_heads, d_k]
fp16 tensor (``memory/mps_memory_pool.py:62``), on a ROCm device.  There is no
CPU path.  Results are fp16 with fp32 arithmetic; the kernel has no context
limit (the reference's kernel holds 512 scores).
"""
from __future__ import annotations

import torch

from . import _native

_workspace: dict[int, torch.Tensor] = {}


def _check(rc: int, what: str) -> None:
    if rc != 0:
        names = {1: "invalid argument", 2: "workspace", 3: "HIP launch failed", 4: "unsupported shape"}
        raise _native.MisError(f"{what} failed: {names.get(rc, rc)}")


def _dev_int32(x, device) -> torch.Tensor:
    return x.to(device=device, dtype=torch.int32).contiguous() if isinstance(x, torch.Tensor) else \
        torch.tensor(x, dtype=torch.int32, device=device)


def fused_attention_fast(pool: torch.Tensor, new_k: torch.Tensor, new_v: torch.Tensor, queries: torch.Tensor,
                         bt_tensor: torch.Tensor, sl_tensor: torch.Tensor, write_info: torch.Tensor,
                         n_heads: int, n_kv_heads: int, d_k: int, block_size: int) -> torch.Tensor:
    """[B, n_heads, d_k] fp16 attention output (kernels/__init__.py:320)."""
    if pool.device.type != "cuda":
        raise _native.MisError("paged attention needs the pool on a ROCm device; there is no CPU path")
    if pool.dtype != torch.float16 or pool.dim() != 5:
        raise ValueError("pool must be a [num_blocks, 2, block_size, n_kv_heads, d_k] float16 tensor")
    nb, two, bs, nkv, dk = pool.shape
    if two != 2 or bs != block_size or nkv != n_kv_heads or dk != d_k or pool.stride(2) != nkv * dk \
            or pool.stride(3) != dk or pool.stride(4) != 1:
        raise ValueError("pool shape / strides do not match block_size, n_kv_heads, d_k")
    lib = _native.load()
    dev = pool.device
    B = bt_tensor.shape[0]
    bt = _dev_int32(bt_tensor, dev)
    sl = _dev_int32(sl_tensor, dev)
    wi = _dev_int32(write_info, dev).view(-1)
    nk = new_k.to(dev, torch.float16).contiguous()
    nv = new_v.to(dev, torch.float16).contiguous()
    q = queries.to(dev, torch.float16).contiguous()
    if nk.shape != (B, n_kv_heads, d_k) or nv.shape != nk.shape or q.shape != (B, n_heads, d_k):
        raise ValueError("new_k / new_v must be [B, n_kv_heads, d_k] and queries [B, n_heads, d_k]")
    out = torch.empty((B, n_heads, d_k), dtype=torch.float16, device=dev)
    max_blocks = bt.shape[1]
    need = int(lib.mis_paged_attention_workspace_bytes(B, n_heads, n_kv_heads, d_k, max_blocks * block_size))
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _workspace.get(idx)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        _workspace[idx] = ws
    rc = lib.mis_paged_attention(pool.data_ptr(), nb, block_size, n_kv_heads, d_k, pool.stride(0), pool.stride(1),
                                 nk.data_ptr(), nv.data_ptr(), q.data_ptr(), bt.data_ptr(), max_blocks, sl.data_ptr(),
                                 wi.data_ptr(), B, n_heads, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                 torch.cuda.current_stream(dev).cuda_stream)
    _check(rc, "mis_paged_attention")
    return out


fused_attention_metal_fast = fused_attention_fast  # the reference's name


def fused_attention(pool, new_k, new_v, queries, block_tables: list[list[int]], seq_lens: list[int],
                    write_blocks: list[int], write_positions: list[int], n_heads: int, n_kv_heads: int,
                    d_k: int, block_size: int) -> torch.Tensor:
    """From Python lists (kernels/__init__.py:371)."""
    B = len(seq_lens)
    max_blocks = max(len(bt) for bt in block_tables)
    bt = torch.zeros(B, max_blocks, dtype=torch.int32)
    for i, row in enumerate(block_tables):
        bt[i, :len(row)] = torch.tensor(row, dtype=torch.int32)
    wi = torch.tensor([[b, p] for b, p in zip(write_blocks, write_positions)], dtype=torch.int32)
    return fused_attention_fast(pool, new_k, new_v, queries, bt, torch.tensor(seq_lens, dtype=torch.int32), wi,
                                n_heads, n_kv_heads, d_k, block_size)


fused_attention_metal = fused_attention


def gather_kv(pool: torch.Tensor, block_tables: torch.Tensor, seq_lens: torch.Tensor,
              max_seq_len: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense [B, max_seq_len, n_kv_heads, d_k] K and V (kernels/__init__.py:279)."""
    if pool.device.type != "cuda":
        raise _native.MisError("gather_kv needs the pool on a ROCm device; there is no CPU path")
    lib = _native.load()
    dev = pool.device
    nb, _, bs, nkv, dk = pool.shape
    bt = _dev_int32(block_tables, dev)
    sl = _dev_int32(seq_lens, dev)
    B = bt.shape[0]
    out_k = torch.empty((B, max_seq_len, nkv, dk), dtype=torch.float16, device=dev)
    out_v = torch.empty_like(out_k)
    rc = lib.mis_gather_kv(pool.data_ptr(), nb, bs, nkv, dk, pool.stride(0), pool.stride(1), bt.data_ptr(),
                           bt.shape[1], sl.data_ptr(), B, max_seq_len, out_k.data_ptr(), out_v.data_ptr(),
                           torch.cuda.current_stream(dev).cuda_stream)
    _check(rc, "mis_gather_kv")
    return out_k, out_v


gather_kv_metal = gather_kv

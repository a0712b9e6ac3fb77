"""CPU restatement of the reference's decode-step paged attention (test
infrastructure only: tests/ and bench.py's cpu_baseline leg use it; the
product path never does).

Reference: the MSL kernel ``fused_attention`` (kernels/__init__.py:79-243)
behind ``fused_attention_metal_fast`` (kernels/__init__.py:320-368), and the
gather ``gather_kv`` (kernels/__init__.py:25-72, :279-311).  Steps, with the
lines each follows:

  write     :128-151   new_k / new_v [B, n_kv_heads, d_k] into the pool at
                       write_info[b] = (block, position), K half and V half
  scores    :158-183   for t < seq_len: s_t = (q . K_t) * scale, K_t read
                       through block_tables[b][t / block_size] at position
                       t % block_size, scale = f32(1 / sqrt(f32(d_k)))
  softmax   :185-205   p_t = exp(s_t - max) / sum
  output    :212-236   out = sum_t p_t V_t, stored as half
  GQA       :114-116   query head h reads KV head h / (n_heads / n_kv_heads)

Here the arithmetic is float64 (the kernel's float32 differs from it by
rounding only); ``out`` is returned unrounded so tests can state their fp16
tolerance.
"""
from __future__ import annotations

import numpy as np


def write_new_kv(pool: np.ndarray, new_k: np.ndarray, new_v: np.ndarray, write_info: np.ndarray) -> np.ndarray:
    """A copy of the pool with the step's K / V written (kernels/__init__.py:128-151)."""
    out = pool.copy()
    for b in range(new_k.shape[0]):
        blk, pos = int(write_info[b, 0]), int(write_info[b, 1])
        out[blk, 0, pos] = new_k[b]
        out[blk, 1, pos] = new_v[b]
    return out


def gather(pool: np.ndarray, block_tables: np.ndarray, seq_lens: np.ndarray, max_seq_len: int):
    """Dense K, V [B, max_seq_len, n_kv_heads, d_k], zero past each length (:25-72)."""
    B = block_tables.shape[0]
    _, _, bs, nkv, dk = pool.shape
    k = np.zeros((B, max_seq_len, nkv, dk), dtype=pool.dtype)
    v = np.zeros_like(k)
    for b in range(B):
        for t in range(min(int(seq_lens[b]), max_seq_len)):
            blk = int(block_tables[b, t // bs])
            k[b, t] = pool[blk, 0, t % bs]
            v[b, t] = pool[blk, 1, t % bs]
    return k, v


def paged_attention(pool: np.ndarray, new_k: np.ndarray, new_v: np.ndarray, queries: np.ndarray,
                    block_tables: np.ndarray, seq_lens: np.ndarray, write_info: np.ndarray, n_heads: int):
    """(out float64 [B, n_heads, d_k], pool after the write)."""
    pool2 = write_new_kv(pool, new_k, new_v, write_info)
    B = queries.shape[0]
    nkv, dk = pool.shape[3], pool.shape[4]
    group = n_heads // nkv
    scale = float(np.float32(1.0) / np.sqrt(np.float32(dk)))
    L = int(seq_lens.max()) if B else 0
    k, v = gather(pool2, block_tables, seq_lens, L)
    out = np.zeros((B, n_heads, dk), dtype=np.float64)
    for b in range(B):
        n = int(seq_lens[b])
        if n == 0:
            continue
        for h in range(n_heads):
            kh = k[b, :n, h // group].astype(np.float64)
            vh = v[b, :n, h // group].astype(np.float64)
            s = kh @ queries[b, h].astype(np.float64) * scale
            e = np.exp(s - s.max())
            out[b, h] = (e / e.sum()) @ vh
    return out, pool2

"""CPU restatement of the greedy decode step's producer and sampler (test
infrastructure only: tests/ and bench.py's cpu_baseline leg use it; the
product path never does).

Reference: the model's lm_head (a bias-free Linear [V, H]) producing
``outputs.logits[:, 0, :]`` in the model dtype (``models/llama_adapter.py:198-207``),
then the sampler's greedy branch ``torch.argmax(logits)``
(``model/sampler.py:32-34``): ties to the lowest index, NaN above every number.

``logits_exact`` is the float64 sum of the exact products (16-bit inputs, so
every product is exact and H = 4096 sums of them stay within float64's
precision to about 1e-16 relative).  ``greedy`` rounds it to float32 and then
to the dtype, as one rounding chain, and takes the argmax.
"""
from __future__ import annotations

import numpy as np


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 (round to nearest even) -> float32; NaN stays NaN."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, r)


def round_dtype(x: np.ndarray, dtype: str) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return round_bf16(x)
    raise ValueError(dtype)


def logits_exact(hidden: np.ndarray, weight: np.ndarray) -> np.ndarray:
    """[B, V] float64; hidden [B, H] and weight [V, H] hold the 16-bit values (as float32)."""
    return hidden.astype(np.float64) @ weight.astype(np.float64).T


def greedy(hidden: np.ndarray, weight: np.ndarray, dtype: str):
    """(ids int64 [B], the exact logits [B, V], the dtype logits [B, V])."""
    ex = logits_exact(hidden, weight)
    lg = round_dtype(ex.astype(np.float32), dtype)
    return np.argmax(lg, axis=1).astype(np.int64), ex, lg


def tolerance(hidden: np.ndarray, weight: np.ndarray, dtype: str) -> np.ndarray:
    """Per row: how far below the exact maximum a sequence's chosen logit may
    lie when the sums are fp32 in another order.  Twice the worst-case fp32
    summation error (H * 2^-24 * sum|x w|, taken at the largest row of |w|)
    plus one dtype ulp at the row's largest magnitude."""
    H = hidden.shape[1]
    absx = np.abs(hidden.astype(np.float64))
    wmax = np.abs(weight.astype(np.float64)).max(axis=0)          # per dim, over the vocabulary
    bound = H * 2.0 ** -24 * (absx @ wmax)
    ex = logits_exact(hidden, weight)
    top = np.abs(ex).max(axis=1)
    ulp = np.ldexp(1.0, np.floor(np.log2(np.maximum(top, 1e-30))).astype(int) - (10 if dtype == "f16" else 7))
    return 2 * bound + ulp

"""CPU restatement of the greedy decode step's producer and sampler (test
infrastructure only: tests/ and bench.py's cpu_baseline leg use it; the
product path never does).

Reference: the model's lm_head (a bias-free Linear [V, H]) producing
``outputs.logits[:, 0, :]`` in the model dtype (``models/llama_adapter.py:198-207``),
then the sampler's greedy branch ``torch.argmax(logits)``
(``model/sampler.py:32-34``): ties to the lowest index, NaN above every number.

``sample`` restates the fused sampling epilogue for temperature-only rows: the
Gumbel-max draw argmax_v(dtype(logit / T) + g_v), exact in distribution
(softmax of the scaled logits, ``model/sampler.py:37, :57-59``); g_v =
-log(-log(u_v)) in float64 from Philox4x32-10 words (numpy, vectorised; pinned
against the C oracle's Random123-checked function in the tests).

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


_M32 = np.uint64(0xFFFFFFFF)


def philox_words(counter: np.ndarray, k0: np.ndarray, k1: np.ndarray) -> np.ndarray:
    """Philox4x32-10 over rows of uint32 counters [N, 4] with keys k0, k1 [N]: [N, 4] uint32."""
    c = [counter[:, i].astype(np.uint64) for i in range(4)]
    k0 = np.asarray(k0, dtype=np.uint64).copy()
    k1 = np.asarray(k1, dtype=np.uint64).copy()
    for r in range(10):
        if r > 0:
            k0 = (k0 + np.uint64(0x9E3779B9)) & _M32
            k1 = (k1 + np.uint64(0xBB67AE85)) & _M32
        p0 = np.uint64(0xD2511F53) * c[0]
        p1 = np.uint64(0xCD9E8D57) * c[2]
        c = [((p1 >> np.uint64(32)) ^ c[1] ^ k0) & _M32, p1 & _M32, ((p0 >> np.uint64(32)) ^ c[3] ^ k1) & _M32, p0 & _M32]
    return np.stack(c, axis=1).astype(np.uint32)


def gumbel(seed: int, request: int, step: int, V: int) -> np.ndarray:
    """float64 [V]: the fused kernel's noise for one draw (include/mis_lmhead.h)."""
    n = (V + 3) // 4
    ctr = np.zeros((n, 4), dtype=np.uint64)
    ctr[:, 0] = np.arange(n, dtype=np.uint64)
    ctr[:, 1] = step & 0xFFFFFFFF
    ctr[:, 2] = request & 0xFFFFFFFF
    ctr[:, 3] = (request >> 32) & 0xFFFFFFFF
    k0 = np.full(n, seed & 0xFFFFFFFF, dtype=np.uint64)
    k1 = np.full(n, ((seed >> 32) ^ (step >> 32)) & 0xFFFFFFFF, dtype=np.uint64)
    w = philox_words(ctr.astype(np.uint32), k0, k1).reshape(-1)[:V]
    u = (w >> 8).astype(np.float64) * 2.0 ** -24
    with np.errstate(divide="ignore"):
        return -np.log(-np.log(u))


def scaled(hidden: np.ndarray, weight: np.ndarray, T: np.ndarray, dtype: str):
    """(exact logits [B, V], y = dtype(dtype logit / T) [B, V] float32)."""
    ex = logits_exact(hidden, weight)
    x = round_dtype(ex.astype(np.float32), dtype)
    with np.errstate(divide="ignore", invalid="ignore"):
        y = round_dtype((x / np.asarray(T, dtype=np.float32)[:, None]).astype(np.float32), dtype)
    return ex, x, y


def sample(hidden: np.ndarray, weight: np.ndarray, dtype: str, T: np.ndarray, seed: int, requests, steps):
    """ids [B] of the fused sampling call: greedy where T = 0, the Gumbel-max
    draw where T > 0, -1 for T < 0 or NaN and for rows whose scaled logits hold
    NaN or +inf or are all -inf.  Also returns z [B, V] (y + g, float64; the
    greedy rows' dtype logits) for the tests' tolerance."""
    ex, x, y = scaled(hidden, weight, T, dtype)
    B, V = x.shape
    ids = np.zeros(B, dtype=np.int64)
    z = np.zeros((B, V), dtype=np.float64)
    for b in range(B):
        t = float(np.float32(T[b]))
        if not t >= 0.0:
            ids[b] = -1
            z[b] = np.nan
            continue
        if t == 0.0:
            z[b] = x[b]
            ids[b] = int(np.argmax(x[b]))
            continue
        yb = y[b].astype(np.float64)
        if np.isnan(yb).any() or np.isposinf(yb).any():
            ids[b] = -1
            z[b] = np.nan
            continue
        z[b] = yb + gumbel(seed, int(requests[b]), int(steps[b]), V)
        ids[b] = -1 if np.isneginf(z[b]).all() else int(np.argmax(z[b]))
    return ids, z, y

"""Pins of the paged-attention oracle (oracle/attention.py) on the CPU:
* against torch's scaled_dot_product_attention in float64 on the gathered,
  GQA-expanded K / V (an independent implementation);
* against a literal float32 restatement of the reference kernel's loops
  (kernels/__init__.py:153-236: sequential dot, max, exp, sum, normalise,
  weighted sum) on small cases, within float32 rounding;
* the pool write and the gather against direct indexing."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as A


def make_case(seed, B, n_heads, n_kv, dk, bs, lens, num_blocks=None):
    rng = np.random.default_rng(seed)
    max_blocks = max((l + bs - 1) // bs for l in lens)
    num_blocks = num_blocks or B * max_blocks + 3
    pool = rng.normal(0, 1, (num_blocks, 2, bs, n_kv, dk)).astype(np.float16)
    perm = rng.permutation(num_blocks)
    bt = np.zeros((B, max_blocks), dtype=np.int32)
    wi = np.zeros((B, 2), dtype=np.int32)
    for b, l in enumerate(lens):
        nblk = (l + bs - 1) // bs
        bt[b, :nblk] = perm[b * max_blocks:b * max_blocks + nblk]
        wi[b] = (bt[b, (l - 1) // bs], (l - 1) % bs)
    q = rng.normal(0, 1, (B, n_heads, dk)).astype(np.float16)
    nk = rng.normal(0, 1, (B, n_kv, dk)).astype(np.float16)
    nv = rng.normal(0, 1, (B, n_kv, dk)).astype(np.float16)
    return pool, nk, nv, q, bt, np.array(lens, dtype=np.int32), wi


@pytest.mark.parametrize("n_heads,n_kv,dk", [(8, 2, 64), (4, 4, 32), (16, 1, 64)])
def test_oracle_matches_sdpa_float64(n_heads, n_kv, dk):
    lens = [1, 15, 16, 17, 70]
    pool, nk, nv, q, bt, sl, wi = make_case(3, len(lens), n_heads, n_kv, dk, 16, lens)
    out, pool2 = A.paged_attention(pool, nk, nv, q, bt, sl, wi, n_heads)
    k, v = A.gather(pool2, bt, sl, int(sl.max()))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(dk)))
    for b, n in enumerate(lens):
        kk = torch.from_numpy(k[b, :n].astype(np.float64)).permute(1, 0, 2)      # [n_kv, n, dk]
        vv = torch.from_numpy(v[b, :n].astype(np.float64)).permute(1, 0, 2)
        kk = kk.repeat_interleave(n_heads // n_kv, dim=0).contiguous()
        vv = vv.repeat_interleave(n_heads // n_kv, dim=0).contiguous()
        qq = torch.from_numpy(q[b].astype(np.float64)).unsqueeze(1)              # [n_heads, 1, dk]
        ref = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, scale=scale)[:, 0]
        np.testing.assert_allclose(out[b], ref.numpy(), rtol=1e-12, atol=1e-12)


def literal_f32(pool2, q, bt, sl, n_heads):
    """The reference kernel's loops in float32, one (sequence, head) at a time."""
    B = q.shape[0]
    nkv, dk, bs = pool2.shape[3], pool2.shape[4], pool2.shape[2]
    group = n_heads // nkv
    scale = np.float32(1.0) / np.sqrt(np.float32(dk))
    out = np.zeros((B, n_heads, dk), dtype=np.float32)
    for b in range(B):
        for h in range(n_heads):
            kvh = h // group
            n = int(sl[b])
            sc = np.zeros(n, dtype=np.float32)
            for t in range(n):
                kr = pool2[bt[b, t // bs], 0, t % bs, kvh].astype(np.float32)
                dot = np.float32(0.0)
                for d in range(dk):
                    dot = np.float32(dot + np.float32(q[b, h, d]) * kr[d])
                sc[t] = dot * scale
            m = sc.max()
            s = np.float32(0.0)
            for t in range(n):
                sc[t] = np.float32(np.exp(sc[t] - m))
                s = np.float32(s + sc[t])
            sc = (sc * (np.float32(1.0) / s)).astype(np.float32)
            for d in range(dk):
                acc = np.float32(0.0)
                for t in range(n):
                    acc = np.float32(acc + sc[t] * np.float32(pool2[bt[b, t // bs], 1, t % bs, kvh, d]))
                out[b, h, d] = acc
    return out


def test_oracle_matches_literal_float32_reference():
    lens = [1, 9, 33]
    pool, nk, nv, q, bt, sl, wi = make_case(5, 3, 4, 2, 16, 8, lens)
    out, pool2 = A.paged_attention(pool, nk, nv, q, bt, sl, wi, 4)
    lit = literal_f32(pool2, q, bt, sl, 4)
    np.testing.assert_allclose(lit, out, rtol=2e-5, atol=2e-6)


def test_write_and_gather_against_indexing():
    lens = [5, 16, 40]
    pool, nk, nv, q, bt, sl, wi = make_case(7, 3, 4, 2, 8, 4, lens)
    pool2 = A.write_new_kv(pool, nk, nv, wi)
    for b in range(3):
        blk, pos = wi[b]
        assert np.array_equal(pool2[blk, 0, pos], nk[b]) and np.array_equal(pool2[blk, 1, pos], nv[b])
    changed = np.argwhere(np.any(pool2 != pool, axis=(1, 3, 4)))
    assert all((blk, pos) in {tuple(x) for x in wi} for blk, pos in changed)
    k, v = A.gather(pool2, bt, sl, 48)
    for b, n in enumerate(lens):
        for t in range(48):
            if t < n:
                assert np.array_equal(k[b, t], pool2[bt[b, t // 4], 0, t % 4])
                assert np.array_equal(v[b, t], pool2[bt[b, t // 4], 1, t % 4])
            else:
                assert not k[b, t].any() and not v[b, t].any()

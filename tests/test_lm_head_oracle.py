"""Pins of the fused lm_head + greedy oracle (oracle/lm_head.py) on the CPU:
* the bfloat16 rounding against torch's own float32 -> bfloat16 conversion;
* the ids against torch's argmax over torch's float64 matmul of the same
  16-bit values, rounded float32 -> dtype (an independent computation of the
  same definition), including ties and NaN;
* the tolerance's arithmetic on a case where it is the only thing that
  separates two logits."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import lm_head as O


def make(seed, B, H, V, dtype):
    g = torch.Generator().manual_seed(seed)
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    x = (torch.randn(B, H, generator=g) * 0.5).to(tdt)
    w = (torch.randn(V, H, generator=g) * 0.05).to(tdt)
    return x, w


def test_round_bf16_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.normal(0, 1, 100000), rng.normal(0, 1e30, 1000), rng.normal(0, 1e-30, 1000),
                        [0.0, -0.0, np.inf, -np.inf, 3.3895314e38, 3.4e38, -3.4e38]]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = O.round_bf16(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.isnan(O.round_bf16(np.array([np.nan], np.float32))).all()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_greedy_matches_torch(dtype):
    x, w = make(1, 6, 256, 3000, dtype)
    ids, ex, lg = O.greedy(x.float().numpy(), w.float().numpy(), dtype)
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    ref = (x.double() @ w.double().T).float().to(tdt)
    assert np.array_equal(ids, torch.argmax(ref, dim=1).numpy())
    assert np.array_equal(lg, ref.float().numpy())


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_greedy_ties_and_nan(dtype):
    x, w = make(2, 3, 64, 500, dtype)
    xs, ws = x.float().numpy(), w.float().numpy()
    ids, _, _ = O.greedy(xs, ws, dtype)
    ws2 = ws.copy()                      # copies of row 0's winner below and above it
    ws2[7] = ws[ids[0]]
    ws2[400] = ws[ids[0]]
    ids2, _, _ = O.greedy(xs, ws2, dtype)
    assert ids2[0] == min(7, ids[0])     # the tie goes to the lowest index
    ws3 = ws.copy()
    ws3[123, 5] = np.nan
    ws3[321, 9] = np.nan
    ids3, _, _ = O.greedy(xs, ws3, dtype)
    assert (ids3 == 123).all()           # NaN above every number, the first NaN
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    ref = (torch.from_numpy(xs).double() @ torch.from_numpy(ws3).double().T).float().to(tdt)
    assert np.array_equal(ids3, torch.argmax(ref, dim=1).numpy())


def test_tolerance_covers_fp32_reordering():
    """The fp32 sum in another order stays within the tolerance of the exact sum."""
    x, w = make(3, 4, 4096, 64, "bf16")
    xs, ws = x.float().numpy(), w.float().numpy()
    ex = O.logits_exact(xs, ws)
    tol = O.tolerance(xs, ws, "bf16")
    rng = np.random.default_rng(0)
    for _ in range(3):
        perm = rng.permutation(4096)
        f32 = np.zeros((4, 64), np.float32)
        for h in perm[:4096]:
            f32 = (f32 + (xs[:, h:h + 1] * ws[:, h][None, :]).astype(np.float32)).astype(np.float32)
        assert (np.abs(f32 - ex) <= tol[:, None] / 2).all()


def test_philox_words_match_c_oracle():
    """The vectorised Philox the sampling oracle uses equals the C oracle's
    function (itself checked against the Random123 known answers)."""
    from oracle import oracle as OR
    rng = np.random.default_rng(0)
    ctr = rng.integers(0, 2 ** 32, (64, 4), dtype=np.uint64).astype(np.uint32)
    key = rng.integers(0, 2 ** 32, (64, 2), dtype=np.uint64).astype(np.uint32)
    got = O.philox_words(ctr, key[:, 0], key[:, 1])
    want = np.stack([OR.philox4x32_10(ctr[i], key[i]) for i in range(64)])
    assert np.array_equal(got, want)


def test_gumbel_max_draws_follow_softmax():
    """The oracle's Gumbel-max draws (many steps of one request) have the
    softmax frequencies of the scaled logits: a chi-square test over 6 tokens."""
    from scipy import stats
    x, w = make(21, 1, 64, 6, "bf16")
    xs, ws = x.float().numpy(), w.float().numpy() * 20
    n = 20000
    T = np.full(n, 0.8, np.float32)
    ids, _, y = O.sample(np.repeat(xs, n, 0), ws, "bf16", T, 7, np.zeros(n, np.int64), np.arange(n))
    p = np.exp(y[0].astype(np.float64) - y[0].max())
    p /= p.sum()
    counts = np.bincount(ids, minlength=6)
    assert stats.chisquare(counts, p * n).pvalue > 1e-4, (counts, p * n)


def test_sample_rows_and_invalid():
    x, w = make(22, 5, 128, 300, "f16")
    xs, ws = x.float().numpy(), w.float().numpy()
    T = np.array([0.0, 1.0, -1.0, np.nan, 0.5], np.float32)
    ids, z, _ = O.sample(xs, ws, "f16", T, 3, np.arange(5), np.zeros(5, np.int64))
    g, _, _ = O.greedy(xs, ws, "f16")
    assert ids[0] == g[0] and ids[2] == -1 and ids[3] == -1
    assert ids[1] == int(np.argmax(z[1])) and ids[4] == int(np.argmax(z[4]))

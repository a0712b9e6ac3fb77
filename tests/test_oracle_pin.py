"""Pin the CPU oracle (oracle/mis_oracle.c) against independent computations.

The reference has no sampler fixtures, so each part of the oracle is pinned
against something that fixes it independently:
* greedy          numpy argmax (first occurrence) and torch.argmax (NaN rule)
* temperature     torch's own ``x / T`` on f32/f16/bf16 tensors
* dtype rounding  numpy float16 and torch bfloat16 conversions
* top-k           np.partition k-th value with ``>=`` and brute force
* 16-bit top-p    torch's own rounding chain, every row accounted for
                  (tests/test_oracle_torch.py)
* fp32 top-p      torch float64 softmax/cumsum; exact Decimal arithmetic on
                  tiny rows
* draw            searchsorted on a float64 CDF; chi-square frequencies
* invariants      monotone in top_p, top-p mask within the top-k mask, rank 0
                  always kept, T = 0 ignores top_k/top_p
* uniforms        Philox4x32-10 known-answer vectors (Random123), the
                  (seed, request, step) -> (key, counter) wiring, and
                  distribution checks (Kolmogorov-Smirnov, lag correlation)
* golden          committed fixtures (tests/golden) and workload digests
"""
from __future__ import annotations

import decimal
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests import harness as H
from vllm_mps_amd import workloads as W

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DT_TORCH = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def torch_tensor(bits: np.ndarray, dtype: str) -> torch.Tensor:
    w = W.Workload("t", dtype, np.ascontiguousarray(bits), np.zeros(1, np.float32), np.zeros(1, np.int32),
                   np.ones(1, np.float32), np.zeros(1, np.float32))
    return w.to_torch("cpu")


def run(w, **kw):
    return O.sample_rows(w.logits, w.dtype, H.params_of(w), want_probs=True, want_keep=True, **kw)


# ----------------------------------------------------------------- greedy

@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_greedy_matches_argmax(dtype):
    w = H.synthetic(dtype, 16, 5000, seed=1, temperature=0.0, top_k=7, top_p=0.3, dup_max=True)
    r = run(w)
    vals = W.bits_to_f32(w.logits, dtype)
    assert np.array_equal(r["ids"], np.argmax(vals, axis=1))
    t = torch_tensor(w.logits, dtype)
    assert np.array_equal(r["ids"], torch.argmax(t, dim=1).numpy())
    # one-hot debug outputs
    assert np.array_equal(r["keep"].sum(1), np.ones(16))


def test_greedy_nan_is_max():
    x = np.array([[1.0, np.nan, 3.0, np.nan, 2.0]], np.float32)
    w = W.Workload("n", "f32", x, np.zeros(1, np.float32), np.zeros(1, np.int32), np.ones(1, np.float32),
                   np.zeros(1, np.float32))
    assert run(w)["ids"][0] == torch.argmax(torch.from_numpy(x[0])).item() == 1


# ------------------------------------------------------------ temperature

@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("T", [0.8, 0.5173, 1.2345678, 1.4999, 7.0, 0.01])
def test_scale_matches_torch_division(dtype, T):
    rng = np.random.default_rng(3)
    bits = W.to_dtype_bits(rng.normal(0, 6, 200_000), dtype)
    y = O.scale(bits, dtype, T)
    ref = (torch_tensor(bits, dtype) / T).float().numpy()
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_round_to_dtype_matches_numpy_and_torch():
    rng = np.random.default_rng(4)
    x = np.concatenate([rng.normal(0, 1, 100_000), rng.normal(0, 1e-6, 50_000),
                        2.0 ** rng.uniform(-30, 17, 50_000)]).astype(np.float32)
    assert np.array_equal(O.round_to(x, "f16"), x.astype(np.float16).astype(np.float32))
    tb = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(O.round_to(x, "bf16"), tb)


# ------------------------------------------------------------------- top-k

@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_topk_mask_closed_form(dtype):
    V = 4000
    ks = [1, 2, 20, 50, 1000, V - 1, V, V + 10]
    w = H.synthetic(dtype, len(ks), V, seed=5, temperature=0.9, top_k=ks, top_p=1.0, dup_max=True, ninf_frac=0.05)
    r = run(w)
    for b, k in enumerate(ks):
        y = O.scale(w.logits[b], dtype, 0.9)
        kk = min(k, V)
        thr = np.partition(y, V - kk)[V - kk]
        expect = (y >= thr) & np.isfinite(y)
        assert np.array_equal(r["keep"][b], expect), k
        assert r["keep"][b].sum() >= min(kk, np.isfinite(y).sum())


def test_topk_brute_force_tiny():
    rng = np.random.default_rng(6)
    for trial in range(200):
        V = int(rng.integers(1, 9))
        x = rng.choice(np.array([-1.0, 0.0, 0.5, 2.0, -np.inf]), V).astype(np.float32)
        k = int(rng.integers(1, V + 2))
        w = W.Workload("t", "f32", x[None, :], np.ones(1, np.float32), np.array([k], np.int32),
                       np.ones(1, np.float32), np.zeros(1, np.float32))
        r = run(w)
        if not np.isfinite(x).any():
            assert r["status"][0] == 2
            continue
        srt = sorted(x, reverse=True)
        thr = srt[min(k, V) - 1]
        assert np.array_equal(r["keep"][0], (x >= thr) & np.isfinite(x))


# --------------------------------------------------------- 16-bit top-p chain
# (pinned row by row against torch's own chain in tests/test_oracle_torch.py)


# ------------------------------------------------------------ fp32 top-p

def test_fp32_topp_matches_torch_float64():
    rng = np.random.default_rng(8)
    for trial in range(30):
        V = int(rng.choice([100, 5000, 128256]))
        T = float(np.float32(rng.uniform(0.5, 1.5)))
        p = float(rng.choice([0.5, 0.9, 0.95, 0.99]))
        k = int(rng.choice([0, 0, 1000]))
        w = H.synthetic("f32", 1, V, seed=200 + trial, temperature=T, top_k=k, top_p=p)
        r = run(w)
        z = torch.from_numpy(w.logits[0]) / T
        if k > 0:
            kth = torch.topk(z, min(k, V)).values[-1]
            z = torch.where(z < kth, torch.full_like(z, float("-inf")), z)
        s, idx = torch.sort(z, descending=True, stable=True)
        pd = torch.softmax(s.double(), -1)
        excl = torch.cumsum(pd, -1) - pd
        removed = excl >= float(np.float32(p))
        keep = torch.zeros(V, dtype=torch.bool)
        keep[idx[~removed & torch.isfinite(s)]] = True
        if not np.array_equal(keep.numpy(), r["keep"][0]):
            assert r["topp_margin"][0] < 1e-12, r["topp_margin"][0]


def test_fp32_topp_exact_decimal_tiny():
    """Exact (50-digit) masses on tiny rows agree with the oracle's x87 sums."""
    decimal.getcontext().prec = 50
    rng = np.random.default_rng(9)
    for trial in range(300):
        V = int(rng.integers(1, 12))
        x = (rng.normal(0, 2, V)).astype(np.float32)
        if trial % 5 == 0:
            x[rng.integers(0, V)] = x.max()  # ties at the top
        T = float(np.float32(rng.uniform(0.5, 1.5)))
        p = float(np.float32(rng.uniform(0.05, 0.99)))
        w = W.Workload("t", "f32", x[None, :], np.full(1, T, np.float32), np.zeros(1, np.int32),
                       np.full(1, p, np.float32), np.zeros(1, np.float32))
        r = run(w)
        y = O.scale(x, "f32", T)
        order = sorted(range(V), key=lambda j: (-float(y[j]), j))
        m = decimal.Decimal(float(y[order[0]]))
        ws = [(decimal.Decimal(float(y[j])) - m).exp() for j in order]
        S = sum(ws)
        thr = decimal.Decimal(float(np.float32(p)))
        E = decimal.Decimal(0)
        keep = np.zeros(V, bool)
        for r_, j in enumerate(order):
            if E >= thr:
                break
            keep[j] = True
            E += ws[r_] / S
        assert np.array_equal(keep, r["keep"][0]), (x, T, p)


# -------------------------------------------------------------------- draw

@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_draw_is_inverse_cdf(dtype):
    rng = np.random.default_rng(10)
    V, B = 3000, 64
    w = H.synthetic(dtype, B, V, seed=11, temperature=1.1, top_k=[0, 30] * 32, top_p=[1.0, 1.0, 0.8, 0.9] * 16,
                    uniforms=rng.random(B, dtype=np.float32))
    r = run(w)
    for b in range(B):
        y = O.scale(w.logits[b], dtype, 1.1).astype(np.float64)
        keep = r["keep"][b]
        wts = np.where(keep, np.exp(y - y[keep].max()), 0.0)
        cdf = np.cumsum(wts)
        tok = int(np.searchsorted(cdf, w.uniform[b] * cdf[-1], side="right"))
        if tok != r["ids"][b]:
            assert r["draw_margin"][b] < 1e-12


def test_draw_frequencies_chi_square():
    """Many uniforms on one small row: token frequencies follow the kept probabilities."""
    V, N = 12, 20000
    rng = np.random.default_rng(12)
    x = np.tile(rng.normal(0, 1, V).astype(np.float32), (N, 1))
    u = rng.random(N, dtype=np.float32)
    w = W.Workload("chi", "f32", x, np.full(N, 0.9, np.float32), np.full(N, 8, np.int32),
                   np.full(N, 0.9, np.float32), u)
    r = O.sample_rows(w.logits, "f32", H.params_of(w), want_probs=True, want_keep=False)
    probs = r["probs"][0].astype(np.float64)
    counts = np.bincount(r["ids"], minlength=V).astype(np.float64)
    nz = probs > 0
    assert counts[~nz].sum() == 0
    exp = probs[nz] / probs[nz].sum() * N
    chi2 = ((counts[nz] - exp) ** 2 / exp).sum()
    from scipy.stats import chi2 as chi2d
    assert chi2 < chi2d.ppf(0.999, int(nz.sum()) - 1), chi2


# -------------------------------------------------------------- invariants

@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_topp_invariants(dtype):
    V = 8000
    ps = [0.01, 0.1, 0.3, 0.5, 0.8, 0.9, 0.95, 0.99, 0.999999, 1.0]
    for seed in range(3):
        w = H.synthetic(dtype, len(ps), V, seed=300 + seed, temperature=1.0, top_k=0, top_p=ps)
        w.logits[:] = w.logits[:1]  # same row, increasing top_p
        r = run(w)
        ks = r["keep"]
        for i in range(len(ps) - 1):
            assert not np.any(ks[i] & ~ks[i + 1]), "mask must grow with top_p"
        y = O.scale(w.logits[0], dtype, 1.0)
        top = int(np.argmax(y))
        assert ks[:, top].all(), "rank 0 is always kept"
    wk = H.synthetic(dtype, 2, V, seed=9, temperature=1.0, top_k=[100, 100], top_p=[1.0, 0.9])
    wk.logits[1] = wk.logits[0]
    rk = run(wk)
    assert not np.any(rk["keep"][1] & ~rk["keep"][0]), "top-p mask within the top-k mask"


def test_greedy_ignores_filters_and_bad_rows():
    V = 500
    w = H.synthetic("f32", 6, V, seed=13, temperature=[0.0, -1.0, 1.0, 1.0, 1.0, 1.0],
                    top_k=[3, 0, -2, 0, 0, 0], top_p=[0.01, 1.0, 1.0, 0.0, 1.0, 1.0])
    f = W.bits_to_f32(w.logits, "f32").copy()
    f[4, :] = -np.inf
    f[5, 3] = np.nan
    w.logits = f
    r = run(w)
    assert r["ids"][0] == int(np.argmax(f[0]))
    assert list(r["status"]) == [0, 1, 1, 1, 2, 2]
    assert list(r["ids"][1:]) == [-1] * 5


def test_bf16_top_p_001_closed_form():
    """top_p = 0.01 keeps rank 0, plus rank 1 iff RN16(fl32(C_1 - p_1)) < RN16(0.01)."""
    V = 128256
    w = W.make_c5(rows=64)
    r = run(w)
    for b in range(64):
        if w.temperature[b] == 0 or w.top_p[b] >= 1.0:
            continue
        y = O.scale(w.logits[b], "bf16", 1.0).astype(np.float64)
        order = np.lexsort((np.arange(V), -y))
        e = np.exp(y[order] - y[order[0]])
        e[~np.isfinite(y[order])] = 0.0
        p16 = O.round_to((e / e.sum()).astype(np.float32), "bf16")
        thr = O.round_to(np.array([0.01], np.float32), "bf16")[0]
        F = np.float32(0.0)
        n = 0
        for i in range(V):
            F = np.float32(F + p16[i])
            C = O.round_to(np.array([F], np.float32), "bf16")[0]
            E = O.round_to(np.array([np.float32(C - p16[i])], np.float32), "bf16")[0]
            if E >= thr:
                break
            n += 1
        assert r["n_kept"][b] == n


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_topp16_near_midpoint_closed_form(dtype):
    """Largest probability 1/S a few 1e-7 above (below) a midpoint M of two
    neighbouring dtype values b1 < b2, top_p = b2: it rounds up to b2 (down
    to b1) exactly when the offset is positive, so rank 0 alone reaches
    top_p (rank 1 is kept as well)."""
    offs = [3e-7, -3e-7, 1e-7, -1e-7, 8e-7, -8e-7]
    w = H.near_midpoint(dtype, 4096, offs, seed=3)
    r = run(w)
    for b, off in enumerate(offs):
        assert r["n_kept"][b] == (1 if off > 0 else 2), (b, off)


# ------------------------------------------------------------------ golden

def test_workload_digests():
    with open(os.path.join(GOLDEN, "digests.json")) as f:
        dig = json.load(f)
    for name in ["C1", "C2", "C3", "C4"]:
        assert W.make(name).digest() == dig[name], name


def test_golden_c1_c2():
    g = np.load(os.path.join(GOLDEN, "c1_c2.npz"))
    for name in ["C1", "C2"]:
        w = W.make(name)
        r = run(w)
        assert np.array_equal(r["ids"], g[f"{name}_ids"])
        assert np.array_equal(r["status"], g[f"{name}_status"])
        bits = np.packbits(r["keep"].astype(np.uint8), axis=1)
        assert np.array_equal(bits, g[f"{name}_keep_bits"])
        kept = (g[f"{name}_kept_rows"], g[f"{name}_kept_cols"])
        assert np.array_equal(r["probs"][kept], g[f"{name}_kept_probs"])


def test_golden_rows_c3_c4():
    with open(os.path.join(GOLDEN, "rows.json")) as f:
        rows = json.load(f)
    for name in ["C3", "C4"]:
        w = W.make(name)
        r = O.sample_rows(w.logits, w.dtype, H.params_of(w), want_keep=True)
        for b, exp in enumerate(rows[name]):
            assert int(r["ids"][b]) == exp["id"], (name, b)
            assert int(r["n_kept"][b]) == exp["n_kept"], (name, b)
            sha = hashlib.sha1(np.packbits(r["keep"][b].astype(np.uint8)).tobytes()).hexdigest()
            assert sha == exp["keep_sha1"], (name, b)


# Philox4x32-10 known answers published with the authors' Random123 library
PHILOX_KAT = [
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
]


def test_philox_known_answers():
    for ctr, key, want in PHILOX_KAT:
        assert O.philox4x32_10(ctr, key).tolist() == want


def test_uniform_wiring():
    """u(seed, request, step) is the first Philox word of counter (step lo,
    step hi, request lo, request hi) under key (seed lo, seed hi), top 24
    bits over 2^24: a swapped field or word order fails here."""
    cases = [(0, 0, 0), (1, 2, 3), (2**64 - 1, 2**63 + 5, 2**40 + 7), (0x0123456789ABCDEF, 9, 2**32)]
    for seed, req, step in cases:
        ctr = [step & 0xFFFFFFFF, step >> 32, req & 0xFFFFFFFF, req >> 32]
        key = [seed & 0xFFFFFFFF, seed >> 32]
        w = int(O.philox4x32_10(ctr, key)[0])
        u = O.uniforms(np.uint64(seed), np.uint64(req), np.uint64(step))
        assert float(u) == (w >> 8) / 2.0**24
    # the fields are not interchangeable
    a = O.uniforms(np.uint64(1), np.uint64(2), np.uint64(3))
    assert a != O.uniforms(np.uint64(1), np.uint64(3), np.uint64(2))
    assert a != O.uniforms(np.uint64(2), np.uint64(1), np.uint64(3))


def test_uniform_distribution():
    """Uniform on [0, 1) across requests and across steps, with no lag-1
    correlation along a request's steps."""
    from scipy import stats
    n = 200000
    by_req = O.uniforms(np.uint64(42), np.arange(n, dtype=np.uint64), np.uint64(0))
    by_step = O.uniforms(np.uint64(42), np.uint64(7), np.arange(n, dtype=np.uint64))
    for u in (by_req, by_step):
        assert u.min() >= 0.0 and u.max() < 1.0
        assert stats.kstest(u, "uniform").pvalue > 1e-4
        assert abs(np.corrcoef(u[:-1], u[1:])[0, 1]) < 0.01
    # 24-bit values: repeats only at the birthday rate (n^2 / 2^25 ~ 1200)
    assert n - np.unique(by_req).size < 2000

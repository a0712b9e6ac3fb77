"""GPU: the fused lm_head + greedy kernel (mis_lm_head_greedy) against the CPU
oracle (oracle/lm_head.py) and against torch's own GEMM + argmax on the GPU.

Bar: the chosen id equals the oracle's, or its exact logit lies within the
stated tolerance of the exact maximum (twice the worst-case fp32 summation
error plus one dtype ulp: the kernel's fp32 additions run in another order
than the oracle's float64 ones, and a near-tie can round either way).  Ties in
the dtype values (duplicated weight rows) go to the lowest index exactly, and
NaN logits win at the first NaN."""
import numpy as np
import pytest
import torch

from oracle import lm_head as O
from tests.test_lm_head_oracle import make
from vllm_mps_amd import lm_head as LH

pytestmark = pytest.mark.gpu

SHAPES = [(1, 64, 1000), (7, 128, 3001), (64, 4096, 32000), (65, 256, 5000), (130, 512, 2049)]


def _check(name, x, w, dtype, device):
    print(f"[lmhead] {name} {dtype} B={x.shape[0]} H={x.shape[1]} V={w.shape[0]}", flush=True)
    got = LH.lm_head_greedy(x.to(device), w.to(device)).cpu().numpy()
    xs, ws = x.float().numpy(), w.float().numpy()
    ids, ex, _ = O.greedy(xs, ws, dtype)
    tol = O.tolerance(xs, ws, dtype)
    rows = np.arange(len(ids))
    assert ((got >= 0) & (got < w.shape[0])).all()
    ok = (got == ids) | (ex[rows, got] >= ex[rows, ids] - tol)
    print(f"[lmhead] {name}: {int((got == ids).sum())}/{len(ids)} equal to the oracle", flush=True)
    assert ok.all(), (np.where(~ok), got[~ok], ids[~ok])
    return got, ids, ex, tol


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("B,H,V", SHAPES)
def test_lm_head_greedy_vs_oracle(B, H, V, dtype, device):
    x, w = make(B * 7 + V, B, H, V, dtype)
    got, ids, _, _ = _check(f"shape", x, w, dtype, device)
    assert (got == ids).mean() >= 0.95


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_lm_head_greedy_vs_torch_gemm(dtype, device):
    """torch's GEMM in the model dtype (the reference's producer) then argmax."""
    x, w = make(11, 64, 4096, 32000, dtype)
    xd, wd = x.to(device), w.to(device)
    ref = torch.argmax(torch.matmul(xd, wd.t().contiguous()), dim=1).cpu().numpy()
    got = LH.lm_head_greedy(xd, wd).cpu().numpy()
    xs, ws = x.float().numpy(), w.float().numpy()
    ex = O.logits_exact(xs, ws)
    tol = O.tolerance(xs, ws, dtype)
    rows = np.arange(64)
    print(f"[lmhead] vs torch {dtype}: {int((got == ref).sum())}/64 equal", flush=True)
    assert ((got == ref) | (np.abs(ex[rows, got] - ex[rows, ref]) <= tol)).all()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_lm_head_greedy_ties_nan_and_strides(dtype, device):
    x, w = make(5, 9, 192, 4099, dtype)
    xs, ws = x.float().numpy(), w.float().numpy()
    ids, _, _ = O.greedy(xs, ws, dtype)
    w2 = w.clone()
    w2[3] = w[int(ids[0])]                 # a duplicate of row 0's winner, lower index
    w2[4098] = w[int(ids[0])]              # and one in the last, partial vocabulary tile
    got = LH.lm_head_greedy(x.to(device), w2.to(device)).cpu().numpy()
    assert got[0] == min(3, int(ids[0]))
    w3 = w.clone()
    w3[2500, 7] = float("nan")
    w3[2600, 1] = float("nan")
    got = LH.lm_head_greedy(x.to(device), w3.to(device)).cpu().numpy()
    assert (got == 2500).all()
    # row strides wider than H (a view into a larger buffer)
    xb = torch.zeros(9, 256, dtype=x.dtype)
    xb[:, :192] = x
    wb = torch.zeros(4099, 200, dtype=w.dtype)
    wb[:, :192] = w
    got = LH.lm_head_greedy(xb.to(device)[:, :192], wb.to(device)[:, :192]).cpu().numpy()
    want = LH.lm_head_greedy(x.to(device), w.to(device)).cpu().numpy()
    assert np.array_equal(got, want)


def _check_sample(name, x, w, dtype, T, seed, req, stp, device):
    print(f"[lmhead-sample] {name} {dtype} B={x.shape[0]} H={x.shape[1]} V={w.shape[0]}", flush=True)
    got = LH.lm_head_sample(x.to(device), w.to(device), torch.from_numpy(T), (seed, req, stp)).cpu().numpy()
    xs, ws = x.float().numpy(), w.float().numpy()
    ids, z, y = O.sample(xs, ws, dtype, T, seed, req, stp)
    same = got == ids
    print(f"[lmhead-sample] {name}: {int(same.sum())}/{len(ids)} equal to the oracle", flush=True)
    bad = ids < 0
    assert np.array_equal(got[bad], ids[bad])
    # elsewhere a different id must be a near-tie of the oracle's maximum:
    # fp32 noise and sums, and a dtype rounding of y the GEMM's order can flip
    ymax = np.nanmax(np.abs(np.where(np.isfinite(y), y, 0)), axis=1)
    ulp = np.ldexp(1.0, np.floor(np.log2(np.maximum(ymax, 1e-30))).astype(int) - (10 if dtype == "f16" else 7))
    zmax = np.nanmax(np.where(np.isfinite(z), np.abs(z), 0), axis=1)
    for b in np.where(~same & ~bad)[0]:
        assert got[b] >= 0 and z[b, got[b]] >= z[b, ids[b]] - (1e-5 * (1 + zmax[b]) + 2 * ulp[b]), b
    return same.mean()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("B,H,V", [(7, 256, 3001), (64, 4096, 32000), (130, 512, 2049)])
def test_lm_head_sample_vs_oracle(B, H, V, dtype, device):
    x, w = make(B + V, B, H, V, dtype)
    rng = np.random.default_rng(B)
    T = rng.choice(np.array([0.0, 0.7, 1.0, 1.3], np.float32), B)
    req = rng.integers(0, 1 << 40, B)
    stp = rng.integers(0, 1000, B)
    assert _check_sample("mixed", x, w, dtype, T, 12345, req, stp, device) >= 0.95


def test_lm_head_sample_greedy_rows_and_invalid(device):
    x, w = make(31, 6, 256, 4099, "bf16")
    T = np.array([0.0, 0.0, 1.0, -1.0, np.nan, 0.9], np.float32)
    got = LH.lm_head_sample(x.to(device), w.to(device), torch.from_numpy(T), (5, np.arange(6), np.zeros(6))).cpu().numpy()
    greedy = LH.lm_head_greedy(x.to(device), w.to(device)).cpu().numpy()
    assert got[0] == greedy[0] and got[1] == greedy[1]
    assert got[3] == -1 and got[4] == -1 and got[2] >= 0 and got[5] >= 0
    w2 = w.clone()
    w2[100, 3] = float("nan")                        # a NaN logit: the sampled rows are invalid
    got = LH.lm_head_sample(x.to(device), w2.to(device), torch.from_numpy(T), (5, np.arange(6), np.zeros(6))).cpu().numpy()
    assert got[2] == -1 and got[5] == -1 and got[0] == 100


def test_lm_head_sample_follows_softmax(device):
    """4096 draws of one request (steps 0..4095) over 8 tokens: the frequencies
    are softmax(y) (chi-square), and every draw equals the oracle's."""
    from scipy import stats
    x, w = make(41, 1, 128, 8, "bf16")
    w = (w.float() * 20).to(torch.bfloat16)
    n = 4096
    xb = x.repeat(n, 1)
    T = np.full(n, 1.0, np.float32)
    got = LH.lm_head_sample(xb.to(device), w.to(device), torch.from_numpy(T), (99, np.zeros(n), np.arange(n))).cpu().numpy()
    ids, _, y = O.sample(xb.float().numpy(), w.float().numpy(), "bf16", T, 99, np.zeros(n, np.int64), np.arange(n))
    assert (got == ids).mean() >= 0.999
    p = np.exp(y[0].astype(np.float64) - y[0].max())
    p /= p.sum()
    print(f"[lmhead-sample] frequencies {np.bincount(got, minlength=8)} expected {np.round(p * n).astype(int)}", flush=True)
    assert stats.chisquare(np.bincount(got, minlength=8), p * n).pvalue > 1e-4


def test_lm_head_sample_device_rng_rows(device):
    """Records built once on the device (rng_rows) give the same draws as the tuple form."""
    x, w = make(51, 9, 256, 3000, "f16")
    T = torch.full((9,), 0.9)
    rng = (77, np.arange(9) * 1000, np.full(9, 5))
    a = LH.lm_head_sample(x.to(device), w.to(device), T, rng)
    b = LH.lm_head_sample(x.to(device), w.to(device), T.to(device), LH.rng_rows(rng, 9, device))
    assert torch.equal(a, b)

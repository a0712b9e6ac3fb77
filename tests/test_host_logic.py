"""Host-compiled checks of the helpers the kernels share (vllm_mps_amd/csrc/mis_common.h).

tests/csrc/host_shim.cpp exposes them through a C ABI; g++ builds it here so
the CPU suite exercises the same source the gfx950 kernels compile.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
F32, F16, BF16 = 0, 1, 2


@pytest.fixture(scope="module")
def shim(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("shim") / "host_shim.so")
    subprocess.run(["g++", "-O2", "-mfma", "-fPIC", "-shared", "-ffp-contract=off", "-o", out,
                    os.path.join(HERE, "csrc", "host_shim.cpp")], check=True)
    L = ctypes.CDLL(out)
    f, u64, i = ctypes.c_float, ctypes.c_uint64, ctypes.c_int
    L.shim_chain_add_n.argtypes = [f, f, u64]; L.shim_chain_add_n.restype = f
    L.shim_chain_naive.argtypes = [f, f, u64]; L.shim_chain_naive.restype = f
    L.shim_chain_E.argtypes = [f, f, i]; L.shim_chain_E.restype = f
    L.shim_rn_dtype.argtypes = [f, i]; L.shim_rn_dtype.restype = f
    L.shim_row_key.argtypes = [f, i]; L.shim_row_key.restype = ctypes.c_uint32
    L.shim_value_of_row_key.argtypes = [ctypes.c_uint32, i]; L.shim_value_of_row_key.restype = f
    L.shim_argmax_key.argtypes = [f]; L.shim_argmax_key.restype = ctypes.c_uint32
    L.shim_rn_dtype_array.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, i]
    L.shim_dexp_array.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    L.shim_div_rcp.argtypes = [f, f]; L.shim_div_rcp.restype = f
    L.shim_div_rcp_sweep.argtypes = [f, u64, u64, u64, ctypes.POINTER(ctypes.c_uint32)]
    L.shim_div_rcp_sweep.restype = u64
    L.shim_philox_uniforms.argtypes = [ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_void_p]
    L.shim_philox4x32_10.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    return L


def bits(x) -> int:
    return int(np.float32(x).view(np.uint32))


def test_chain_add_n_matches_sequential_float(shim):
    """Closed-form run addition == one IEEE float addition per element,
    including ties to even and binade crossings."""
    rng = np.random.default_rng(0)
    for it in range(20000):
        F = 0.0 if rng.random() < 0.1 else float(np.float32(2.0 ** rng.uniform(-30, 1)))
        mode = it % 4
        if mode == 0:
            p = float(np.float32(2.0 ** rng.uniform(-40, 0)))
        elif mode == 1:  # bf16-representable p
            p = float(np.array([np.float32(2.0 ** rng.uniform(-30, -1)).view(np.uint32) & 0xFFFF0000],
                               np.uint32).view(np.float32)[0])
        elif mode == 2:  # exact half-ulp ties relative to F
            if F == 0:
                F = float(np.float32(2.0 ** rng.uniform(-10, 0)))
            e = np.frexp(np.float32(F))[1] - 1
            p = float(np.float32(2.0 ** (e - 23) * (rng.integers(0, 6) + 0.5)))
        else:
            p = float(np.float32(F * rng.uniform(0, 3))) if F > 0 else float(np.float32(2.0 ** rng.uniform(-20, 0)))
        n = int(rng.integers(1, 2000))
        a, b = shim.shim_chain_add_n(F, p, n), shim.shim_chain_naive(F, p, n)
        assert bits(a) == bits(b), (F, p, n, a, b)


def test_chain_add_n_subnormal_and_large_n(shim):
    tiny = float(np.float32(1e-44))
    assert bits(shim.shim_chain_add_n(0.0, tiny, 1000)) == bits(shim.shim_chain_naive(0.0, tiny, 1000))
    for p in [1e-8, 3e-8, 6e-8, 1.2e-7]:
        a = shim.shim_chain_add_n(0.5, p, 200000)
        b = shim.shim_chain_naive(0.5, p, 200000)
        assert bits(a) == bits(b), p


@pytest.mark.parametrize("dt,name", [(F16, "f16"), (BF16, "bf16")])
def test_rn_dtype_matches_reference_conversions(shim, dt, name):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.normal(0, 1, 50000), rng.normal(0, 1e-5, 20000), 2.0 ** rng.uniform(-40, 20, 20000),
                        [0.0, -0.0, np.inf, -np.inf, 65504.0, 65520.0, 6e-8, 3e-8]]).astype(np.float32)
    y = np.empty_like(x)
    shim.shim_rn_dtype_array(x.ctypes.data, y.ctypes.data, x.size, dt)
    ref = x.astype(np.float16).astype(np.float32) if name == "f16" else \
        torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    with np.errstate(invalid="ignore"):
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_chain_E_is_torch_subtraction(shim):
    rng = np.random.default_rng(2)
    for dt, tdt in [(F16, torch.float16), (BF16, torch.bfloat16)]:
        C = torch.from_numpy(rng.uniform(0, 1, 5000).astype(np.float32)).to(tdt)
        p = torch.from_numpy((rng.uniform(0, 1, 5000) ** 4).astype(np.float32)).to(tdt)
        E = (C - p).float().numpy()
        for i in range(0, 5000, 7):
            # chain_E(F, p) rounds F to the dtype first; pass an F that already is C
            got = shim.shim_chain_E(float(C[i].float()), float(p[i].float()), dt)
            assert bits(got) == bits(E[i])


@pytest.mark.parametrize("dt", [F32, F16, BF16])
def test_row_key_orders_like_values(shim, dt):
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.normal(0, 10, 3000), [0.0, -0.0, np.inf, -np.inf, 1e-30, -1e-30]]).astype(np.float32)
    if dt != F32:
        y = np.empty_like(x)
        shim.shim_rn_dtype_array(x.ctypes.data, y.ctypes.data, x.size, dt)
        x = y
    keys = np.array([shim.shim_row_key(float(v), dt) for v in x], np.uint64)
    order_k = np.argsort(keys, kind="stable")
    assert np.all(np.diff(x[order_k]) >= 0)
    # equal values <=> equal keys (+0 and -0 included)
    eq_v = x[:, None] == x[None, :]
    eq_k = keys[:, None] == keys[None, :]
    sub = slice(0, 400)
    assert np.array_equal(eq_v[sub, sub], eq_k[sub, sub])
    back = np.array([shim.shim_value_of_row_key(int(k), dt) for k in keys], np.float32)
    assert np.array_equal(back, x)  # -0.0 == 0.0 compares equal
    if dt != F32:
        assert np.all(keys & 0xFFFF == 0)


def test_argmax_key_nan_first(shim):
    assert shim.shim_argmax_key(float("nan")) == 0xFFFFFFFF
    assert shim.shim_argmax_key(float("inf")) < 0xFFFFFFFF
    assert shim.shim_argmax_key(1.0) > shim.shim_argmax_key(-1.0)


def test_dexp_relative_error(shim):
    """The float64 exp of the fp32 top-p masses against x87 extended
    precision (64-bit significand): relative error below DEXP_REL_ERR = 1e-15
    wherever the result is normal, exact at 0, zero at -inf."""
    rng = np.random.default_rng(7)
    d = np.concatenate([
        -rng.exponential(3.0, 200000), -rng.uniform(0, 708, 200000), -rng.uniform(0, 1e-3, 20000),
        -np.arange(0, 700, 0.0078125),  # table boundaries j/64 and binade edges
        np.array([0.0, -0.0, -1e-300, -708.0, -744.9, -745.0, -800.0, -np.inf]),
    ]).astype(np.float64)
    out = np.empty_like(d)
    shim.shim_dexp_array(d.ctypes.data, out.ctypes.data, d.size)
    ref = np.exp(d.astype(np.longdouble))
    normal = ref >= np.longdouble(2.2250738585072014e-308)
    rel = np.abs((out[normal].astype(np.longdouble) - ref[normal]) / ref[normal])
    assert float(rel.max()) < 1e-15, float(rel.max())
    sub = ~normal & (d > -745.0)
    assert np.all(np.abs(out[sub].astype(np.longdouble) - ref[sub]) <= np.longdouble(2.0 ** -1074))
    assert np.all(out[d == 0.0] == 1.0)
    assert np.all(out[d <= -745.0] == 0.0)


# temperatures of the configs (C2 0.8, C3's seeded U[0.5, 1.5] draws, the edge
# tests' extremes) and a few with long reciprocal expansions
def _config_temperatures():
    from vllm_mps_amd import workloads as W
    c3 = W.make_c3().temperature
    return sorted({0.8, 1.0, 0.7, 1.3, 0.9, 1.1, 1.2, 0.6, 1.4, 0.001, 0.01, 50.0, 7.0, 0.5173, 1.2345678,
                   1.4999, 0.3, 2.0, *map(float, c3[::16])})


def test_div_rcp_exhaustive_binade(shim):
    """div_rcp (Markstein reciprocal division, run on every element the chunk
    pass scales) == IEEE x / T bit for bit.  For a fixed T the quotient's
    rounding depends only on x's significand (a power-of-two factor of x is
    exact), so every float in [1, 2) covers every normal x whose quotient
    stays inside div_rcp_safe's range; outside it div_rcp divides."""
    first = ctypes.c_uint32(0)
    lo, hi = 0x3F800000, 0x40000000  # [1, 2)
    for T in _config_temperatures():
        bad = shim.shim_div_rcp_sweep(ctypes.c_float(T), lo, hi, 1, ctypes.byref(first))
        assert bad == 0, (T, bad, hex(first.value))


def test_div_rcp_every_binade_strided(shim):
    """Every sign, exponent, subnormal and special value (stride 7 over all
    2^32 bit patterns) at two temperatures, including the range edges where
    div_rcp falls back to the division."""
    first = ctypes.c_uint32(0)
    for T in (0.8, 1.2345678):
        bad = shim.shim_div_rcp_sweep(ctypes.c_float(T), 0, 1 << 32, 7, ctypes.byref(first))
        assert bad == 0, (T, bad, hex(first.value))


# Philox4x32-10 known answers published with the authors' Random123 library
# (counter words, key words, output words)
PHILOX_KAT = [
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
]


def test_device_philox_known_answers(shim):
    for ctr, key, want in PHILOX_KAT:
        c, k = np.array(ctr, np.uint32), np.array(key, np.uint32)
        out = np.zeros(4, np.uint32)
        shim.shim_philox4x32_10(c.ctypes.data, k.ctypes.data, out.ctypes.data)
        assert out.tolist() == want


def test_device_uniforms_match_oracle(shim):
    """The kernels' uniform (mis_common.h) against the oracle's restatement,
    bit for bit, over triples that set every word of the key and counter."""
    from oracle import oracle as O
    rng = np.random.default_rng(11)
    n = 20000
    seed, req, step = (rng.integers(0, 2**64 - 1, n, dtype=np.uint64, endpoint=True) for _ in range(3))
    step[:100] = np.arange(100, dtype=np.uint64)  # small counters, as a new request has
    req[100:200] = 0
    got = np.zeros(n, np.float32)
    shim.shim_philox_uniforms(n, seed.ctypes.data, req.ctypes.data, step.ctypes.data, got.ctypes.data)
    want = O.uniforms(seed, req, step)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))

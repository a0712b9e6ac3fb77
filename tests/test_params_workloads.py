"""SamplingParams (mirrors the reference's validation), host-side parameter
packing, workload generators and the bench.py contract -- all CPU-only."""
from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from vllm_mps_amd import SamplingParams
from vllm_mps_amd import workloads as W
from vllm_mps_amd.sampler import host_row_params, pack_params

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_sampling_params_validation():
    """Same cases as the reference's tests/test_sequence.py:55-64."""
    with pytest.raises(ValueError):
        SamplingParams(temperature=-1.0)
    with pytest.raises(ValueError):
        SamplingParams(top_k=-1)
    with pytest.raises(ValueError):
        SamplingParams(top_p=0.0)
    with pytest.raises(ValueError):
        SamplingParams(max_tokens=0)
    with pytest.raises(ValueError):
        SamplingParams(top_p=1.5)
    sp = SamplingParams()
    assert (sp.temperature, sp.top_k, sp.top_p, sp.max_tokens, sp.stop_sequences) == (1.0, 0, 1.0, 128, [])


def test_host_row_params_rounding_rules():
    ps = [SamplingParams(temperature=0.8, top_k=50, top_p=0.9), SamplingParams(temperature=0.0),
          SamplingParams(top_p=1.0 - 1e-9), SamplingParams(temperature=1e-50)]
    h16 = host_row_params(ps, torch.float16)
    f = h16.view(np.float32)
    assert f[0, 0] == np.float32(0.8) and h16[0, 1] == 50 and f[0, 2] == np.float32(0.9)
    assert f[1, 0] == 0.0
    # top_p < 1 rounding to 1.0f stays active for 16-bit logits (threshold RN16 = 1.0)
    assert f[2, 2] < 1.0 and np.float16(f[2, 2]) == np.float16(1.0)
    # ... and is a no-op for fp32 logits
    assert host_row_params(ps, torch.float32).view(np.float32)[2, 2] == 1.0
    # a positive temperature that underflows f32 cannot be divided by: flagged
    assert np.isnan(f[3, 0])


def test_pack_params_layout():
    T = torch.tensor([0.5, 1.0]); k = torch.tensor([3, 0]); p = torch.tensor([0.9, 1.0]); u = torch.tensor([0.25, 0.75])
    pk = pack_params(T, k, p, u)
    assert pk.dtype == torch.int32 and pk.shape == (2, 4) and pk.is_contiguous()
    rec = pk.numpy().view(np.float32)
    assert rec[0, 0] == 0.5 and pk[0, 1] == 3 and rec[0, 2] == np.float32(0.9) and rec[1, 3] == 0.75


def test_c3_row_mix():
    w = W.make("C3")
    assert w.shape == (256, 128256) and w.dtype == "f32"
    kinds = W.c3_row_kinds()
    assert np.bincount(kinds).tolist() == [64, 128, 64]
    assert set(np.unique(w.top_k).tolist()) == {0, 20, 1000}
    assert set(np.unique(w.top_p).tolist()) == {np.float32(1.0), np.float32(0.95), np.float32(0.5)}
    assert w.temperature.min() >= 0.5 and w.temperature.max() <= 1.5
    # zipf rows are -1.1 ln(rank) under a permutation
    z = int(np.nonzero(kinds == 2)[0][0])
    srt = np.sort(w.logits[z])[::-1]
    assert np.allclose(srt[:5], -1.1 * np.log(np.arange(1, 6)), atol=1e-6)


def test_c5_edge_structure():
    w = W.make_c5(rows=128)
    vals = W.bits_to_f32(w.logits, "bf16")
    assert np.all(np.isneginf(vals).sum(1) == 12826)
    dup = [r for r in W.c5_duplicate_rows() if r < 128]
    for r in dup:
        fin = vals[r][np.isfinite(vals[r])]
        assert (fin == fin.max()).sum() >= 2
    full_dup = W.c5_duplicate_rows()
    assert len(full_dup) == 51 and len(set(full_dup)) == 51
    cls = W.c5_row_classes()
    assert set(cls[full_dup].tolist()) == set(range(len(W.C5_CLASSES)))  # duplicates in every class
    # the generated params follow the class table
    for r in range(128):
        t, k, p = W.C5_CLASSES[cls[r]]
        assert w.temperature[r] == np.float32(t) and w.top_p[r] == np.float32(p)
        assert w.top_k[r] == (128256 if k < 0 else k)


def test_bench_refuses_multi_gpu():
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True)
    assert out.returncode == 2
    assert "one GPU only" in out.stderr


def test_row_kinds_hint():
    """Host-side row-kind hint: fp32 top-p rows (T > 0, top-k off, top_p < 1)
    versus every other row; 16-bit batches have no fp32 top-p rows; GENERIC
    marks the others the generic row pass serves (1024 < k' < V, 16-bit
    top-p without top-k)."""
    import torch
    from vllm_mps_amd.sampler import KIND_GENERIC, KIND_OTHER, KIND_TOPP32, row_kinds
    V = 100
    assert row_kinds([1.0], [0], [0.9], V, torch.float32) == KIND_TOPP32
    assert row_kinds([1.0], [V], [0.9], V, torch.float32) == KIND_TOPP32      # k >= V is off
    assert row_kinds([1.0], [20], [0.9], V, torch.float32) == KIND_OTHER       # small-k branch
    assert row_kinds([0.0], [0], [0.9], V, torch.float32) == KIND_OTHER        # greedy
    assert row_kinds([1.0], [0], [1.0], V, torch.float32) == KIND_OTHER        # top-p off
    assert row_kinds([1.0, 0.0], [0, 0], [0.5, 1.0], V, torch.float32) == KIND_TOPP32 | KIND_OTHER
    assert row_kinds([1.0], [0], [0.9], V, torch.float16) == KIND_OTHER | KIND_GENERIC
    assert row_kinds([1.0], [20], [0.9], V, torch.bfloat16) == KIND_OTHER
    assert row_kinds([1.0], [0], [1.0], V, torch.bfloat16) == KIND_OTHER
    assert row_kinds([1.0], [50], [1.0], 5000, torch.float32) == KIND_OTHER
    assert row_kinds([1.0], [2000], [1.0], 5000, torch.float32) == KIND_OTHER | KIND_GENERIC
    assert row_kinds([0.0], [2000], [0.5], 5000, torch.float16) == KIND_OTHER  # greedy ignores the filters
    assert row_kinds([], [], [], V, torch.float32) == 0


def test_rng_rows_records():
    from vllm_mps_amd.sampler import rng_rows
    r = rng_rows(3, 7, [10, 11, 12], 0)
    assert r.dtype == np.uint64 and r.shape == (3, 3)
    assert r[:, 0].tolist() == [7, 7, 7] and r[:, 1].tolist() == [10, 11, 12] and r[:, 2].tolist() == [0, 0, 0]
    big = rng_rows(1, 2**64 - 1, 2**63, 2**40)
    assert big.tolist() == [[2**64 - 1, 2**63, 2**40]]
    with pytest.raises(ValueError):
        rng_rows(2, 0, [1, 2, 3], 0)      # wrong length
    with pytest.raises(ValueError):
        rng_rows(1, -1, 0, 0)             # negative
    with pytest.raises(ValueError):
        rng_rows(1, 0, 2**64, 0)          # beyond 64 bits


def test_step_sampler_checks_without_gpu():
    import torch
    from vllm_mps_amd import StepSampler, SamplingParams
    s = StepSampler(seed=5)
    assert s.sample_step(torch.zeros((0, 10)), [], {}) == []
    with pytest.raises(ValueError):
        s.sample_step(torch.zeros((2, 10)), [1], {})            # rows != ids
    with pytest.raises(ValueError):
        s.sample_step(torch.zeros((2, 10)), [4, 4], {})         # duplicate id
    with pytest.raises(ValueError):
        StepSampler(seed=-1)
    assert s.step_of(3) == 0
    s.release(3)  # unknown ids are fine

"""GPU: the per-request device generator (mis_fill_uniforms) and the
engine-shaped batched caller (StepSampler) against the CPU oracle.

* mis_fill_uniforms writes exactly the oracle's Philox uniforms into the
  parameter records, bit for bit, and touches nothing else;
* StepSampler.sample_step over several decode steps gives the oracle's tokens
  for uniforms (seed, request = sequence id, step), on fp32 and fp16 batches;
* a sequence's token does not depend on the batch it is sampled in;
* a rejected row raises as the reference does and advances no step counter.

Every case prints its name before touching the GPU so a failing run names it.
"""
import numpy as np
import pytest
import torch

from oracle import compare as C
from oracle import oracle as O
from tests import harness as H
from vllm_mps_amd import SamplingParams, StepSampler, _native
from vllm_mps_amd import workloads as W

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B", [1, 255, 256, 257, 5000])
def test_fill_uniforms_match_oracle(B, device):
    print(f"[rng] fill_uniforms B={B}", flush=True)
    rng = np.random.default_rng(B)
    state = rng.integers(0, 2**64 - 1, (B, 3), dtype=np.uint64, endpoint=True)
    state[: min(B, 10), 2] = np.arange(min(B, 10), dtype=np.uint64)
    params = np.zeros((B, 4), dtype=np.int32)
    params[:, 0] = rng.integers(-2**31, 2**31 - 1, B)
    params[:, 1] = rng.integers(-2**31, 2**31 - 1, B)
    params[:, 2] = rng.integers(-2**31, 2**31 - 1, B)
    params[:, 3] = -1
    dp = torch.from_numpy(params).to(device)
    ds = torch.from_numpy(state.view(np.int64)).to(device)
    _native.fill_uniforms(dp.data_ptr(), ds.data_ptr(), B, torch.cuda.current_stream(device).cuda_stream)
    got = dp.cpu().numpy()
    want = O.uniforms(state[:, 0], state[:, 1], state[:, 2])
    assert np.array_equal(got[:, 3].view(np.float32).view(np.uint32), want.view(np.uint32))
    assert np.array_equal(got[:, :3], params[:, :3])


def _params_map(w, seq_ids):
    return {int(s): SamplingParams(temperature=float(w.temperature[i]), top_k=int(w.top_k[i]),
                                   top_p=float(w.top_p[i])) for i, s in enumerate(seq_ids)}


def _oracle_step(w, seed, seq_ids, steps):
    u = O.uniforms(np.uint64(seed), np.asarray(seq_ids, dtype=np.uint64), np.asarray(steps, dtype=np.uint64))
    w2 = W.Workload(w.name, w.dtype, w.logits, w.temperature, w.top_k, w.top_p, u)
    return w2, H.run_oracle(w2, debug=False)


@pytest.mark.parametrize("name", ["C3[:64]", "C2"])
def test_step_sampler_matches_oracle(name, device):
    w = W.make_c3().rows(np.arange(64)) if name == "C3[:64]" else W.make("C2")
    B = w.shape[0]
    seq_ids = [int(x) for x in np.random.default_rng(3).choice(10**9, B, replace=False)]
    table = _params_map(w, seq_ids)
    ss = StepSampler(seed=2024)
    logits = w.to_torch(device)
    seen = []
    for step in range(3):
        print(f"[engine] {name} step {step}", flush=True)
        ids = ss.sample_step(logits, seq_ids, table)
        w2, o = _oracle_step(w, 2024, seq_ids, [step] * B)
        g = dict(ids=np.array(ids, dtype=np.int64), status=np.zeros(B, dtype=np.int32))
        rep = C.compare(w.dtype, H.params_of(w2), g, o)
        print(f"[engine] {name} step {step}: {rep.summary()}", flush=True)
        assert rep.ok, rep.summary()
        seen.append(ids)
    assert all(ss.step_of(s) == 3 for s in seq_ids)
    # stochastic rows draw fresh uniforms each step
    stoch = np.nonzero(w.temperature > 0)[0]
    assert any(seen[0][i] != seen[1][i] or seen[1][i] != seen[2][i] for i in stoch)


def test_step_sampler_batch_independence(device):
    """A sequence's token depends on its own logits, parameters, seed and
    step, not on the other rows of the batch or their order."""
    w = W.make_c3().rows(np.arange(48))
    seq_ids = list(range(100, 148))
    table = _params_map(w, seq_ids)
    print("[engine] batch independence: full batch", flush=True)
    full = StepSampler(seed=9).sample_step(w.to_torch(device), seq_ids, table)
    sub = np.random.default_rng(1).permutation(48)[:17]
    print("[engine] batch independence: permuted subset", flush=True)
    part = StepSampler(seed=9).sample_step(w.rows(sub).to_torch(device), [seq_ids[i] for i in sub], table)
    assert part == [full[i] for i in sub]


def test_step_sampler_error_rows(device):
    """A row whose scaled logits hold NaN raises RuntimeError, as
    torch.multinomial does in the reference loop, and no counter advances."""
    w = H.synthetic("f32", 4, 3000, seed=8, temperature=1.0, top_k=0, top_p=0.9)
    x = w.logits.copy()
    x[2, 17] = np.nan
    w = W.Workload("nan-row", "f32", x, w.temperature, w.top_k, w.top_p, w.uniform)
    seq_ids = [5, 6, 7, 8]
    ss = StepSampler(seed=1)
    print("[engine] NaN row raises", flush=True)
    with pytest.raises(RuntimeError):
        ss.sample_step(w.to_torch(device), seq_ids, _params_map(w, seq_ids))
    assert all(ss.step_of(s) == 0 for s in seq_ids)
    # the same step without the bad row succeeds and advances its rows only
    print("[engine] the other rows", flush=True)
    ok = [0, 1, 3]
    ids = ss.sample_step(w.rows(ok).to_torch(device), [seq_ids[i] for i in ok], _params_map(w, seq_ids))
    assert len(ids) == 3 and all(0 <= t < 3000 for t in ids)
    assert [ss.step_of(s) for s in seq_ids] == [1, 1, 0, 1]

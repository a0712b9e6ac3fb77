"""GPU tests through the drop-in surface: ``Sampler.sample`` /
``sample_batch`` (model/sampler.py:18,62), ``Sampler.sample_rows`` (the
engine's per-row loop, engine/llm_engine.py:339-345, as one call) and the
row status -> exception mapping, each compared with the oracle on the same
uniforms; and config C5 at its full batch against tests/golden/rows.json.

Every case prints its name before touching the GPU.
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from oracle import compare as C
from oracle import oracle as O
from tests import harness as H
from vllm_mps_amd import Sampler, SamplingParams
from vllm_mps_amd import workloads as W

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _params_list(w):
    return [SamplingParams(temperature=float(w.temperature[b]), top_k=int(w.top_k[b]), top_p=float(w.top_p[b]))
            for b in range(w.shape[0])]


def _compare_ids(w, ids, status):
    o = H.run_oracle(w, debug=False)
    rep = C.compare(w.dtype, H.params_of(w), dict(ids=np.asarray(ids), status=np.asarray(status)), o)
    assert rep.ok, rep.summary()
    return rep


def _gen_uniforms(seed, B, device):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.rand(B, device=device, dtype=torch.float32, generator=g)


def test_sample_rows_c3_per_row_params(device):
    print("[facade] sample_rows C3 per-row params, explicit uniforms", flush=True)
    w = W.make_c3()
    s = Sampler()
    status = torch.empty(w.shape[0], dtype=torch.int32, device=device)
    ids = s.sample_rows(w.to_torch(device), _params_list(w), torch.from_numpy(w.uniform).to(device),
                        status_out=status)
    torch.cuda.synchronize(device)
    _compare_ids(w, ids.cpu().numpy(), status.cpu().numpy())


@pytest.mark.parametrize("name", ["C2", "C4"])
def test_sample_batch_shared_params(name, device):
    print(f"[facade] sample_batch {name}", flush=True)
    w = W.make(name)
    g = torch.Generator(device=device)
    g.manual_seed(1234)
    sp = SamplingParams(temperature=float(w.temperature[0]), top_k=int(w.top_k[0]), top_p=float(w.top_p[0]))
    toks = Sampler(generator=g).sample_batch(w.to_torch(device), sp)
    assert isinstance(toks, list) and all(isinstance(t, int) for t in toks)
    # the same uniforms, drawn again from an identically seeded generator
    u = _gen_uniforms(1234, w.shape[0], device).cpu().numpy()
    w.uniform = u
    _compare_ids(w, toks, np.zeros(w.shape[0], np.int32))


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_sample_single_rows(dtype, device):
    print(f"[facade] sample() stochastic rows {dtype}", flush=True)
    V = 30000
    T = [1.0, 0.7, 1.3, 0.9, 1.1]
    k = [0, 40, 0, 1000, 0]
    p = [0.9, 1.0, 0.5, 0.95, 1.0]
    w = H.synthetic(dtype, len(T), V, seed=55, temperature=T, top_k=k, top_p=p)
    t = w.to_torch(device)
    for b in range(len(T)):
        g = torch.Generator(device=device)
        g.manual_seed(700 + b)
        tok = Sampler(generator=g).sample(t[b], SamplingParams(temperature=T[b], top_k=k[b], top_p=p[b]))
        assert isinstance(tok, int)
        one = w.rows(np.array([b]))
        one.uniform = _gen_uniforms(700 + b, 1, device).cpu().numpy()
        _compare_ids(one, [tok], [0])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_status_exceptions(dtype, device):
    print(f"[facade] status -> exception mapping {dtype}", flush=True)
    V = 500
    w = H.synthetic(dtype, 1, V, seed=5, temperature=1.0, top_k=0, top_p=1.0)
    x = w.to_torch(device)[0]
    s = Sampler()
    # NaN temperature passes SamplingParams' check; torch's multinomial raises
    with pytest.raises(RuntimeError):
        s.sample(x, SamplingParams(temperature=float("nan")))
    # a positive temperature whose f32 is 0: x / 0 -> inf / NaN, multinomial raises
    with pytest.raises(RuntimeError):
        s.sample(x, SamplingParams(temperature=1e-50))
    # nothing left to sample
    ninf = torch.full_like(x, float("-inf"))
    with pytest.raises(RuntimeError):
        s.sample(ninf, SamplingParams(temperature=1.0))
    # parameters mutated past SamplingParams' validation
    sp = SamplingParams(temperature=1.0)
    sp.top_k = -1
    with pytest.raises(ValueError):
        s.sample(x, sp)
    sp = SamplingParams(temperature=1.0)
    sp.top_p = 0.0
    with pytest.raises(ValueError):
        s.sample_batch(torch.stack([x, x]), sp)
    # greedy ignores the filters and still works on the same sampler
    assert s.sample(x, SamplingParams(temperature=0.0, top_k=3, top_p=0.2)) == int(torch.argmax(x).item())
    # per-row statuses through sample_rows: ids -1 where a row is rejected
    st = torch.empty(4, dtype=torch.int32, device=device)
    bad = SamplingParams(temperature=1.0)
    bad.top_k = -2
    ids = s.sample_rows(torch.stack([x, ninf, x, x]), [SamplingParams(), SamplingParams(), bad,
                                                         SamplingParams(temperature=float("nan"))],
                        status_out=st)
    assert st.tolist() == [0, 2, 1, 2], st.tolist()
    assert ids.tolist()[1:] == [-1, -1, -1]


def test_config_c5_full_batch(device):
    """C5 (bf16 [1024, 128256]) at its full batch: ids, kept counts and keep
    masks against the committed per-row golden (tests/golden/rows.json),
    and ids against the oracle's draw (margin exemption)."""
    print("[facade] C5 full batch vs golden rows", flush=True)
    w = W.make_c5()
    g = H.run_gpu(w, device, debug=True, probs=False)
    with open(os.path.join(GOLDEN, "rows.json")) as f:
        rows = json.load(f)["C5"]
    assert len(rows) == w.shape[0]
    o = O.sample_rows(w.logits, w.dtype, H.params_of(w), want_keep=False)
    for b, exp in enumerate(rows):
        assert int(g["status"][b]) == 0, b
        kb = g["keep"][b]
        assert int(kb.sum()) == exp["n_kept"], (b, int(kb.sum()), exp["n_kept"])
        assert hashlib.sha1(np.packbits(kb.astype(np.uint8)).tobytes()).hexdigest() == exp["keep_sha1"], b
        if int(g["ids"][b]) != exp["id"]:
            assert float(o["draw_margin"][b]) < C.DRAW_MARGIN, (b, int(g["ids"][b]), exp["id"])

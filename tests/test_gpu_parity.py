"""GPU parity: the HIP sampler (through the C ABI) against the CPU oracle.

Every case prints its name before touching the GPU so a failing run names it.
"""
import numpy as np
import pytest

from tests import harness as H
from vllm_mps_amd import workloads as W

pytestmark = pytest.mark.gpu


def _run(name, w, device, **kw):
    print(f"[parity] {name} dtype={w.dtype} shape={w.shape}", flush=True)
    rep = H.check(w, device, **kw)
    print(f"[parity] {name}: {rep.summary()}", flush=True)
    assert rep.ok, rep.summary()
    return rep


@pytest.mark.parametrize("name", ["C1", "C2", "C4"])
def test_config_small(name, device):
    _run(name, W.make(name), device)


def test_config_c3_full(device):
    rep = _run("C3", W.make_c3(), device)
    # the headline config must not lean on the fp32 margin exemption
    assert len(rep.exempt_mask) == 0, rep.exempt_mask


@pytest.mark.parametrize("kinds", [0, 1, 2, 3])
def test_row_kind_hints(kinds, device):
    """The row-kind hint only selects launches: C3's first 64 rows (both
    kinds) give the oracle's results under every hint, wrong ones included."""
    w = W.make_c3().rows(np.arange(64))
    _run(f"C3[:64] kinds={kinds}", w, device, kinds=kinds)


def test_config_c5_subset(device):
    w = W.make_c5(rows=96)
    _run("C5[:96]", w, device)


def test_config_c5_duplicate_rows(device):
    w = W.make_c5()
    rows = np.array(W.c5_duplicate_rows())
    _run("C5[dup]", w.rows(rows), device)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("V", [1, 2, 3, 31, 33, 257, 1000, 2049, 5003])
def test_ragged_vocab(dtype, V, device):
    B = 6
    w = H.synthetic(dtype, B, V, seed=V, temperature=[0.0, 1.0, 0.7, 1.3, 1.0, 0.9],
                    top_k=[0, 0, 3, 0, 1, 50], top_p=[1.0, 1.0, 1.0, 0.8, 0.5, 0.9])
    _run(f"ragged V={V}", w, device)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_unaligned_stride(dtype, device):
    w = H.synthetic(dtype, 5, 4001, seed=11, temperature=[0.0, 1.0, 0.8, 1.2, 1.0],
                    top_k=[0, 0, 20, 0, 7], top_p=[1.0, 0.9, 1.0, 0.95, 0.6])
    print("[parity] unaligned stride", flush=True)
    rep = H.check(w, device, stride_pad=3)
    assert rep.ok, rep.summary()


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_edge_params(dtype, device):
    V = 3000
    T = [1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 0.001, 50.0, 1.0, 1.0]
    k = [1, V, V + 5, 0, 0, 1000, 0, 0, 0, 2]
    p = [1.0, 1.0, 1.0, 1e-3, 0.999999, 1.0, 0.9, 0.9, 1e-30, 0.01]
    w = H.synthetic(dtype, len(T), V, seed=5, temperature=T, top_k=k, top_p=p, dup_max=True)
    _run("edge params", w, device)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_bad_rows(dtype, device):
    V = 700
    w = H.synthetic(dtype, 6, V, seed=9, temperature=[-1.0, 1.0, 1.0, float("nan"), 1.0, 1.0],
                    top_k=[0, -3, 0, 0, 0, 0], top_p=[1.0, 1.0, 0.0, 1.0, 1.0, 1.0])
    raw = w.logits.copy()
    f = W.bits_to_f32(raw, dtype)
    f[4, :] = -np.inf          # nothing to sample
    f[5, 17] = np.nan          # NaN logit
    w.logits = W.to_dtype_bits(f.astype(np.float64), dtype)
    _run("bad rows", w, device)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_neg_inf_and_ties(dtype, device):
    V = 20000
    w = H.synthetic(dtype, 8, V, seed=21, temperature=[1.0, 0.0, 1.0, 1.0, 0.8, 1.0, 1.0, 1.0],
                    top_k=[0, 0, 1, 5, 0, V, 100, 0], top_p=[0.5, 1.0, 1.0, 0.9, 0.01, 0.01, 0.7, 1.0],
                    ninf_frac=0.3, dup_max=True)
    _run("neg inf + ties", w, device)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_large_k_generic_path(dtype, device):
    V = 40000
    w = H.synthetic(dtype, 4, V, seed=31, temperature=[1.0, 0.9, 1.1, 1.0],
                    top_k=[5000, 20000, 1500, 39999], top_p=[1.0, 0.9, 0.95, 0.5])
    _run("large k", w, device)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_candidate_overflow(dtype, device):
    # every element equal: each chunk's top-k' ties exceed the candidate buffer
    V = 50000
    w = H.synthetic(dtype, 3, V, seed=41, temperature=1.0, top_k=[10, 3, 1000], top_p=[1.0, 0.5, 0.9])
    w.logits[:] = w.logits[:, :1]
    _run("candidate overflow", w, device)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_topk_ties_past_survivor_list(dtype, device):
    # N(0, 3^2) rows at T = 0.8: the 1000th / 1024th largest 16-bit value is
    # tied with enough others that more than 1024 elements survive top-k, so
    # the small-k path hands the row to the radix descent
    w = H.synthetic(dtype, 4, 128256, seed=77, temperature=0.8, top_k=[1000, 1024, 1000, 1024],
                    top_p=[1.0, 1.0, 0.9, 1.0])
    _run("top-k ties past the survivor list", w, device)


@pytest.mark.parametrize("seed", range(6))
def test_fuzz(seed, device):
    rng = np.random.default_rng(1000 + seed)
    dtype = ["f32", "f16", "bf16"][seed % 3]
    B = int(rng.integers(1, 24))
    V = int(rng.integers(50, 60000))
    T = np.where(rng.random(B) < 0.15, 0.0, rng.uniform(0.3, 2.0, B))
    k = np.where(rng.random(B) < 0.4, 0, rng.integers(1, 3000 if dtype == "f32" else 1025, B))
    p = np.where(rng.random(B) < 0.4, 1.0, rng.uniform(0.05, 0.999, B))
    w = H.synthetic(dtype, B, V, seed=seed, temperature=T, top_k=k, top_p=p,
                    scale=float(rng.uniform(0.5, 6.0)), ninf_frac=float(rng.choice([0.0, 0.0, 0.2])))
    _run(f"fuzz {seed}", w, device)


def test_workspace_reuse_across_shapes(device):
    """One Sampler (one workspace) across shapes and dtypes: the per-row
    control words the kernel leaves at zero must serve every later call."""
    from vllm_mps_amd.sampler import Sampler
    s = Sampler()
    cases = [("f32", 40, 70000), ("bf16", 7, 128256), ("f32", 300, 9000), ("f16", 3, 20000), ("f32", 40, 70000)]
    for rep_i in range(2):
        for i, (dtype, B, V) in enumerate(cases):
            w = H.synthetic(dtype, B, V, seed=100 + i, temperature=np.linspace(0.0, 1.5, B),
                            top_k=np.where(np.arange(B) % 3 == 0, 20, 0), top_p=np.where(np.arange(B) % 2, 0.9, 1.0))
            print(f"[parity] reuse {rep_i}/{i} {dtype} B={B} V={V}", flush=True)
            rep = H.check(w, device, debug=(i % 2 == 0), sampler=s)
            assert rep.ok, rep.summary()


@pytest.mark.parametrize("scale", [0.05, 0.4, 3.0])
def test_topp_f32_refinement_rounds(scale, device):
    """fp32 top-p rows whose cut bin holds many elements (narrow logits):
    exercises the histogram round, the collect round and their overflow exits."""
    B, V = 12, 128256
    p = [0.95, 0.5, 0.9, 0.99, 0.3, 0.7, 0.95, 0.5, 0.9, 0.99, 0.3, 0.7]
    w = H.synthetic("f32", B, V, seed=int(scale * 100), temperature=[1.0, 0.7, 1.3] * 4, top_k=0, top_p=p,
                    scale=scale)
    _run(f"topp rounds scale={scale}", w, device)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_large_vocab_64_per_thread(dtype, device):
    """V = 2,200,000 needs more than 256 chunks of 8192: the chunk pass runs
    64 elements per thread (chunks of 16384) and so do the top-p passes."""
    B, V = 5, 2_200_000
    w = H.synthetic(dtype, B, V, seed=55, temperature=[0.0, 1.0, 1.0, 0.8, 1.2], top_k=[0, 0, 100, 0, 0],
                    top_p=[1.0, 0.9, 1.0, 1.0, 0.5] if dtype == "f32" else [1.0, 1.0, 0.9, 1.0, 1.0], scale=2.0)
    _run(f"large V {dtype}", w, device, debug=False)


def test_topp_f32_all_equal(device):
    """Every logit equal: staging and window buffers overflow, the row falls
    back to the re-read path; the keep set is the lowest indices."""
    B, V = 3, 100000
    w = H.synthetic("f32", B, V, seed=5, temperature=1.0, top_k=0, top_p=[0.5, 0.9, 0.01])
    w.logits[:] = w.logits[:, :1]
    _run("topp all equal", w, device)


def test_repeat_deterministic(device):
    """The same batch sampled repeatedly with one workspace gives identical ids."""
    from vllm_mps_amd.sampler import Sampler
    s = Sampler()
    w = W.make_c3()
    first = None
    for it in range(4):
        print(f"[parity] repeat C3 {it}", flush=True)
        g = H.run_gpu(w, device, debug=False, sampler=s)
        if first is None:
            first = g
        assert np.array_equal(g["ids"], first["ids"]) and np.array_equal(g["status"], first["status"])


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("V", [4096, 50000])
def test_topp16_rounding_near_midpoint(dtype, V, device):
    """fp16/bf16 top-p rows whose largest probability sits within a few 1e-7
    of a rounding midpoint: the chunk pass's float32-exp S cannot decide that
    rounding, so the row pass must take S exactly before walking the chain."""
    offs = [3e-7, -3e-7, 6e-7, -6e-7, 1e-7, -1e-7, 8e-7, -8e-7, 2e-6, -2e-6]
    w = H.near_midpoint(dtype, V, offs, seed=11 + V)
    _run(f"topp16 near midpoint V={V}", w, device)

"""CPU emulation of the HIP kernels against the oracle (no GPU needed).

tests/emu builds the product's kernel sources as host C++ (AddressSanitizer,
array-bounds checks) and runs every workgroup on the CPU with exact wave64
semantics.  Each case below runs the real launch sequence (mis_sample_ex)
and compares ids, status, keep masks and probabilities with the oracle, to
the same bar as the GPU parity tests; any out-of-bounds global or LDS access,
a shuffle from an inactive lane or a barrier not every lane reaches aborts
the run and fails the test.

The fp16/bf16 radix-descent cases (1 024 < k' < V, candidate overflow, and
top-k ties past the 1 024-survivor LDS list) are the ones a single-launch
build of the kernels once faulted on; they run here before they run on a GPU.
"""
import numpy as np
import pytest

from oracle import compare as C
from tests import harness as H


def _emu(w, **kw):
    from tests.emu import runner
    return runner.run(w, **kw)


def _check(name, w, kinds=7, side=True, noalloc=False):
    print(f"[emu] {name} dtype={w.dtype} shape={w.shape}", flush=True)
    g = _emu(w, kinds=kinds, side=side, noalloc=noalloc)
    rep = C.compare(w.dtype, H.params_of(w), g, H.run_oracle(w))
    print(f"[emu] {name}: {rep.summary()}", flush=True)
    assert rep.ok, rep.summary()
    return rep


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_emu_large_k_generic_path(dtype):
    V = 40000
    w = H.synthetic(dtype, 4, V, seed=31, temperature=[1.0, 0.9, 1.1, 1.0],
                    top_k=[5000, 20000, 1500, 39999], top_p=[1.0, 0.9, 0.95, 0.5])
    _check("large k", w)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_emu_candidate_overflow(dtype):
    V = 50000
    w = H.synthetic(dtype, 3, V, seed=41, temperature=1.0, top_k=[10, 3, 1000], top_p=[1.0, 0.5, 0.9])
    w.logits[:] = w.logits[:, :1]
    _check("candidate overflow", w)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_emu_topk_ties_past_survivor_list(dtype):
    # N(0, 3^2) rows at T = 0.8: the 1000th / 1024th largest 16-bit value is
    # tied with enough others that more than 1024 elements survive top-k
    w = H.synthetic(dtype, 4, 128256, seed=77, temperature=0.8, top_k=[1000, 1024, 1000, 1024],
                    top_p=[1.0, 1.0, 0.9, 1.0])
    o = H.run_oracle(w)
    assert int(o["n_kept"][1]) > 1024 and int(o["n_kept"][3]) > 1024, o["n_kept"]
    g = _emu(w)
    rep = C.compare(w.dtype, H.params_of(w), g, o)
    assert rep.ok, rep.summary()


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_emu_mixed_modes(dtype):
    V = 9000
    T = [0.0, 1.0, 0.7, 1.3, 1.0, 0.9, 1.0, 1.2]
    k = [0, 0, 20, 0, 1, 50, 2000, 0]
    p = [1.0, 1.0, 1.0, 0.8, 0.5, 0.9, 0.7, 0.95]
    w = H.synthetic(dtype, len(T), V, seed=3, temperature=T, top_k=k, top_p=p, ninf_frac=0.1, dup_max=True)
    _check("mixed", w)
    # hints that leave kinds out, and one stream without a context: the same
    # results through the fallback phases
    for kinds in (3, 2, 1):
        _check(f"mixed kinds={kinds}", w, kinds=kinds)
    _check("mixed one stream", w, side=False)
    _check("mixed one stream kinds=3", w, kinds=3, side=False)
    # the allocation-free entry point: the static scratch instead of a workspace
    _check("mixed noalloc", w, noalloc=True)


def test_emu_config_c2():
    from vllm_mps_amd import workloads as W
    _check("C2", W.make("C2"))


def test_emu_fp32_topp_passes():
    # fp32 top-p rows beside other rows: the split chunk pass and the k_tp_*
    # passes; the row-kind hint both ways
    V = 20000
    w = H.synthetic("f32", 6, V, seed=12, temperature=[1.0, 0.6, 1.4, 1.0, 0.0, 1.0],
                    top_k=[0, 0, 0, 20, 0, 0], top_p=[0.95, 0.5, 0.9, 1.0, 1.0, 0.999])
    _check("fp32 top-p split", w, kinds=3)
    g = _emu(w, kinds=2)  # wrong hint: every row on the generic paths, same results
    rep = C.compare(w.dtype, H.params_of(w), g, H.run_oracle(w))
    assert rep.ok, rep.summary()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_emu_t16_ties_across_chunks(dtype):
    """16-bit top-p rows whose logits take a few dozen values, each held by
    thousands of elements over many chunks: the cut falls inside a run that
    spans chunks (the tie index resolved in one chunk, or at a chunk's end)."""
    from vllm_mps_amd import workloads as W
    B, V = 6, 60000
    rng = np.random.default_rng(21)
    x = np.round(rng.normal(0.0, 1.0, (B, V)) * 4.0) / 4.0
    w = W.Workload("ties", dtype, W.to_dtype_bits(x, dtype), np.full(B, 1.0, np.float32),
                   np.zeros(B, np.int32), np.array([0.3, 0.5, 0.7, 0.9, 0.95, 0.99], np.float32),
                   rng.random(B, dtype=np.float32))
    _check("t16 ties", w)


def test_emu_t16_wide_key_range_defers():
    """fp16 values spread over more binades than the key histogram holds,
    with nearly equal masses: the cut lies under the histogram's range and
    the generic path serves the row, with the same results."""
    from vllm_mps_amd import workloads as W
    B, V = 3, 20000
    rng = np.random.default_rng(22)
    x = np.exp2(rng.uniform(-14.0, -6.0, (B, V)))
    w = W.Workload("wide", "f16", W.to_dtype_bits(x, "f16"), np.full(B, 1.0, np.float32), np.zeros(B, np.int32),
                   np.array([0.9, 0.5, 0.999], np.float32), rng.random(B, dtype=np.float32))
    _check("t16 wide range", w)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_emu_topp16_both_paths(dtype):
    """The same 16-bit top-p rows in a batch of 256 rows (each row one
    workgroup: the K_PROBE probe, then the generic path) and in a batch of 64
    (the t16 passes): both give the oracle's results."""
    B, V = 256, 3000
    rng = np.random.default_rng(23)
    p = rng.choice([0.01, 0.3, 0.9, 0.99], B).astype(np.float32)
    w = H.synthetic(dtype, B, V, seed=24, temperature=rng.uniform(0.5, 1.5, B).astype(np.float32), top_k=0, top_p=p)
    _check("topp16 B=256", w)
    _check("topp16 B=64", w.rows(np.arange(64)))

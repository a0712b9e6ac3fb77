"""GPU: decode-step paged attention (mis_paged_attention, mis_gather_kv)
against the CPU oracle (oracle/attention.py).

Bar: the fp16 output within one fp16 ulp of the float64 oracle
(|gpu - oracle| <= 2^-10 |oracle| + 2^-14 max|V|: the kernel's float32
sums differ from float64 by rounding only, and the result is rounded to
fp16 once); the pool after the call equal to the oracle's bit for bit (the
new K / V written at write_info, nothing else touched); the gather bit-exact.

Every case prints its name before touching the GPU so a failing run names it.
"""
import numpy as np
import pytest
import torch

from oracle import attention as A
from tests.test_attention_oracle import make_case
from vllm_mps_amd import attention as VA

pytestmark = pytest.mark.gpu

SHAPES = {  # (n_heads, n_kv_heads, d_k)
    "tinyllama": (32, 4, 64),
    "llama8b": (32, 8, 128),
    "mha256": (8, 8, 256),
    "gqa16": (16, 1, 64),
    "g8": (64, 8, 128),
    "g3": (12, 4, 128),
    "g16d256": (16, 1, 256),
}


def _run(name, device, n_heads, n_kv, dk, lens, bs=16, seed=0):
    print(f"[attn] {name} heads={n_heads}/{n_kv} d_k={dk} lens={lens[:6]}{'...' if len(lens) > 6 else ''}",
          flush=True)
    pool, nk, nv, q, bt, sl, wi = make_case(seed, len(lens), n_heads, n_kv, dk, bs, lens)
    want, pool_want = A.paged_attention(pool, nk, nv, q, bt, sl, wi, n_heads)
    dpool = torch.from_numpy(pool).to(device)
    out = VA.fused_attention_fast(dpool, torch.from_numpy(nk).to(device), torch.from_numpy(nv).to(device),
                                  torch.from_numpy(q).to(device), torch.from_numpy(bt), torch.from_numpy(sl),
                                  torch.from_numpy(wi), n_heads, n_kv, dk, bs)
    torch.cuda.synchronize(device)
    got = out.float().cpu().numpy().astype(np.float64)
    vmax = float(np.abs(pool.astype(np.float32)).max())
    err = np.abs(got - want)
    bound = 2.0 ** -10 * np.abs(want) + 2.0 ** -14 * vmax
    worst = float((err / bound).max())
    print(f"[attn] {name}: max err / bound = {worst:.3f}", flush=True)
    assert (err <= bound).all(), worst
    assert np.array_equal(dpool.cpu().numpy().view(np.uint16), pool_want.view(np.uint16))
    return dpool, bt, sl


@pytest.mark.parametrize("shape", list(SHAPES))
def test_attention_short_contexts(shape, device):
    n_heads, n_kv, dk = SHAPES[shape]
    _run(shape, device, n_heads, n_kv, dk, [1, 2, 15, 16, 17, 100, 255, 256], seed=1)


@pytest.mark.parametrize("shape", ["tinyllama", "llama8b"])
def test_attention_split_contexts(shape, device):
    """Contexts over 256 tokens: several workgroups per (sequence, KV head)
    and the merge; lengths around the split boundaries."""
    n_heads, n_kv, dk = SHAPES[shape]
    _run(shape + " long", device, n_heads, n_kv, dk, [257, 511, 512, 513, 1000, 2048, 3, 4093], seed=2)


@pytest.mark.parametrize("B,ctx", [(8, 700), (16, 1500), (64, 1024)])
def test_attention_split_sizes(B, ctx, device):
    """Splits of 64, 128 and 256 tokens (the split shrinks while the grid is
    small): random lengths up to ctx over llama8b's shape."""
    lens = [int(x) for x in np.random.default_rng(B).integers(1, ctx + 1, B)]
    lens[0] = ctx
    _run(f"split B={B} ctx={ctx}", device, 32, 8, 128, lens, seed=B)


@pytest.mark.parametrize("bs", [32, 8, 24])
def test_attention_block_size_and_batch(bs, device):
    """Block sizes: 32 (whole 16-token tiles in a block), 8 and 24 (tiles
    across blocks; 24 is no power of two)."""
    lens = [int(x) for x in np.random.default_rng(4).integers(1, 700, 40)]
    _run(f"bs{bs} B=40", device, 32, 8, 128, lens, bs=bs, seed=4)


def test_gather_bit_exact(device):
    lens = [1, 16, 17, 300]
    pool, nk, nv, q, bt, sl, wi = make_case(9, len(lens), 8, 2, 64, 16, lens)
    print("[attn] gather", flush=True)
    dk_, dv_ = VA.gather_kv(torch.from_numpy(pool).to(device), torch.from_numpy(bt), torch.from_numpy(sl), 320)
    k, v = A.gather(pool, bt, sl, 320)
    assert np.array_equal(dk_.cpu().numpy().view(np.uint16), k.view(np.uint16))
    assert np.array_equal(dv_.cpu().numpy().view(np.uint16), v.view(np.uint16))


def test_attention_list_entry_point(device):
    """fused_attention (the reference's list-based wrapper) equals the tensor entry point."""
    lens = [5, 40]
    pool, nk, nv, q, bt, sl, wi = make_case(11, 2, 8, 2, 64, 16, lens)
    want, _ = A.paged_attention(pool, nk, nv, q, bt, sl, wi, 8)
    print("[attn] list entry point", flush=True)
    out = VA.fused_attention(torch.from_numpy(pool).to(device), torch.from_numpy(nk).to(device),
                             torch.from_numpy(nv).to(device), torch.from_numpy(q).to(device),
                             [list(r[:(l + 15) // 16]) for r, l in zip(bt, lens)], lens, list(wi[:, 0]),
                             list(wi[:, 1]), 8, 2, 64, 16)
    got = out.float().cpu().numpy()
    assert np.abs(got - want).max() <= 2.0 ** -10 * np.abs(want).max() + 1e-3

"""mis_sample_noalloc (no workspace argument: the library's static per-device
scratch serves instead) against mis_sample on the same inputs, through the C
ABI: bit-identical token ids, row statuses, post-filter probabilities and keep
masks, on calls in a row whose later inputs are smaller, so each call runs
over the scratch contents the one before left behind.

Every case prints its name before touching the GPU so a failing run names it.
"""
import numpy as np
import pytest
import torch

from tests import harness as H
from vllm_mps_amd import _native
from vllm_mps_amd import workloads as W
from vllm_mps_amd.sampler import dtype_code, pack_params

pytestmark = pytest.mark.gpu


def _inputs(w, device):
    t = w.to_torch(device)
    packed = pack_params(torch.from_numpy(w.temperature).to(device), torch.from_numpy(w.top_k).to(device),
                         torch.from_numpy(w.top_p).to(device), torch.from_numpy(w.uniform).to(device))
    return t, packed


def _call(w, device, noalloc, kinds=_native.KIND_ALL):
    B, V = w.shape
    t, packed = _inputs(w, device)
    ids = torch.full((B,), -9, dtype=torch.int64, device=device)
    status = torch.full((B,), -7, dtype=torch.int32, device=device)
    probs = torch.full((B, V), -1.0, dtype=torch.float32, device=device)
    keep = torch.zeros((B, (V + 31) // 32), dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    args = (t.data_ptr(), dtype_code(t.dtype), B, V, t.stride(0), packed.data_ptr(), ids.data_ptr(),
            status.data_ptr(), probs.data_ptr(), keep.data_ptr())
    if noalloc:
        _native.sample_noalloc(*args, stream, kinds)
    else:
        ws = torch.empty(_native.workspace_bytes(B, V, dtype_code(t.dtype)), dtype=torch.uint8, device=device)
        _native.sample(*args, ws.data_ptr(), ws.numel(), stream, kinds=kinds)
    torch.cuda.synchronize(device)
    return dict(ids=ids.cpu().numpy(), status=status.cpu().numpy(), probs=probs.cpu().numpy(),
                keep=keep.cpu().numpy())


def _same(name, w, device, kinds=_native.KIND_ALL):
    print(f"[noalloc] {name} dtype={w.dtype} shape={w.shape} kinds={kinds}", flush=True)
    ref = _call(w, device, noalloc=False, kinds=kinds)
    got = _call(w, device, noalloc=True, kinds=kinds)
    for key in ("ids", "status", "keep"):
        np.testing.assert_array_equal(got[key], ref[key], err_msg=f"{name}: {key}")
    # bit-identical probabilities (NaN-safe comparison of the bit patterns)
    np.testing.assert_array_equal(got["probs"].view(np.uint32), ref["probs"].view(np.uint32),
                                  err_msg=f"{name}: probs")
    assert (got["status"] >= 0).all() and (got["ids"] >= -1).all()
    print(f"[noalloc] {name}: ok", flush=True)


def test_noalloc_matches_workspace_entry(device):
    # the headline shape (fp32 B = 256, V = 128256), then smaller calls over
    # the scratch the larger one left behind
    _same("C3", W.make_c3(), device)
    _same("C5[:96]", W.make_c5(rows=96), device)
    _same("C3[:64] kinds=1", W.make_c3().rows(np.arange(64)), device, kinds=_native.KIND_TOPP32)
    w = H.synthetic("f16", 6, 2049, seed=3, temperature=[0.0, 1.0, 0.7, 1.3, 1.0, 0.9],
                    top_k=[0, 0, 3, 0, 1, 50], top_p=[1.0, 1.0, 1.0, 0.8, 0.5, 0.9])
    _same("ragged f16", w, device)


def test_noalloc_rejects_shapes_beyond_scratch(device):
    B, V = 1024, 128256
    assert _native.workspace_bytes(B, V, _native.DTYPE_F32) > _native.SCRATCH_BYTES
    x = torch.zeros((B, V), dtype=torch.float32, device=device)
    params = torch.zeros((B, 4), dtype=torch.int32, device=device)
    ids = torch.full((B,), -9, dtype=torch.int64, device=device)
    print("[noalloc] oversize shape is rejected before any launch", flush=True)
    with pytest.raises(_native.MisError, match="scratch"):
        _native.sample_noalloc(x.data_ptr(), _native.DTYPE_F32, B, V, V, params.data_ptr(), ids.data_ptr(), None,
                               None, None, torch.cuda.current_stream(device).cuda_stream)
    torch.cuda.synchronize(device)
    assert (ids.cpu().numpy() == -9).all()

"""Shared GPU/oracle runners for the parity tests and __graft_entry__.smoke()."""
from __future__ import annotations

import numpy as np

from oracle import compare as C
from oracle import oracle as O
from vllm_mps_amd import workloads as W


def params_of(w: W.Workload) -> np.ndarray:
    return O.make_params(w.temperature, w.top_k, w.top_p, w.uniform)


def run_gpu(w: W.Workload, device, debug: bool = True, stride_pad: int = 0, sampler=None, kinds=None) -> dict:
    import torch
    from vllm_mps_amd.sampler import Sampler, pack_params

    B, V = w.shape
    t = w.to_torch(device)
    if stride_pad:
        big = torch.zeros((B, V + stride_pad), dtype=t.dtype, device=device)
        big[:, :V] = t
        t = big[:, :V]
    packed = pack_params(torch.from_numpy(w.temperature).to(device), torch.from_numpy(w.top_k).to(device),
                         torch.from_numpy(w.top_p).to(device), torch.from_numpy(w.uniform).to(device))
    status = torch.full((B,), -7, dtype=torch.int32, device=device)
    probs = torch.full((B, V), -1.0, dtype=torch.float32, device=device) if debug else None
    keep = torch.zeros((B, (V + 31) // 32), dtype=torch.int32, device=device) if debug else None
    s = Sampler() if sampler is None else sampler
    ids = s.sample_packed(t, packed, status_out=status, probs_out=probs, keep_out=keep, kinds=kinds)
    torch.cuda.synchronize(device)
    out = dict(ids=ids.cpu().numpy(), status=status.cpu().numpy())
    if debug:
        out["probs"] = probs.cpu().numpy()
        out["keep"] = C.unpack_keep(keep.cpu().numpy(), V)
    return out


def run_oracle(w: W.Workload, debug: bool = True) -> dict:
    return O.sample_rows(w.logits, w.dtype, params_of(w), want_probs=debug, want_keep=debug)


def check(w: W.Workload, device, debug: bool = True, stride_pad: int = 0, sampler=None, kinds=None) -> C.Report:
    g = run_gpu(w, device, debug=debug, stride_pad=stride_pad, sampler=sampler, kinds=kinds)
    o = run_oracle(w, debug=debug)
    return C.compare(w.dtype, params_of(w), g, o)


def synthetic(dtype: str, B: int, V: int, seed: int, temperature, top_k, top_p, scale=3.0,
              ninf_frac=0.0, dup_max=False, uniforms=None, name="synthetic") -> W.Workload:
    """Small seeded workload with explicit per-row params (broadcast)."""
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, scale, (B, V))
    if ninf_frac > 0:
        for b in range(B):
            n = int(round(ninf_frac * V))
            if n:
                x[b, rng.choice(V, n, replace=False)] = -np.inf
    bits = W.to_dtype_bits(x, dtype)
    if dup_max:
        vals = W.bits_to_f32(bits, dtype)
        for b in range(B):
            if V > 1:
                a = int(np.argmax(vals[b]))
                j = int(rng.integers(0, V))
                if j != a and np.isfinite(vals[b, j]):
                    bits[b, j] = bits[b, a]
    bc = lambda v, dt: np.ascontiguousarray(np.broadcast_to(np.asarray(v, dtype=dt), (B,)))
    u = rng.random(B, dtype=np.float32) if uniforms is None else bc(uniforms, np.float32)
    return W.Workload(name, dtype, bits, bc(temperature, np.float32), bc(top_k, np.int32),
                      bc(top_p, np.float32), u)

"""Shared GPU/oracle runners for the parity tests and __graft_entry__.smoke()."""
from __future__ import annotations

import numpy as np

from oracle import compare as C
from oracle import oracle as O
from vllm_mps_amd import workloads as W


def params_of(w: W.Workload) -> np.ndarray:
    return O.make_params(w.temperature, w.top_k, w.top_p, w.uniform)


def run_gpu(w: W.Workload, device, debug: bool = True, stride_pad: int = 0, sampler=None, kinds=None,
            probs: bool = True) -> dict:
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
    pr = torch.full((B, V), -1.0, dtype=torch.float32, device=device) if debug and probs else None
    keep = torch.zeros((B, (V + 31) // 32), dtype=torch.int32, device=device) if debug else None
    s = Sampler() if sampler is None else sampler
    ids = s.sample_packed(t, packed, status_out=status, probs_out=pr, keep_out=keep, kinds=kinds)
    torch.cuda.synchronize(device)
    out = dict(ids=ids.cpu().numpy(), status=status.cpu().numpy())
    if pr is not None:
        out["probs"] = pr.cpu().numpy()
    if keep is not None:
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


def near_midpoint(dtype: str, V: int, offsets, seed: int = 7, top_p_upper: bool = True) -> W.Workload:
    """Rows (T = 1, top-p) whose largest probability 1/S lies at a relative
    offset (one per row, e.g. +3e-7 / -3e-7) from a midpoint between two
    neighbouring values of the 16-bit dtype, so its rounding depends on S
    beyond what a float32-exp estimate of S (relative error ~1e-7) fixes.
    The max is 0 (weight 1); the rest start at or below -6 (forty of them at
    -60) and mass is added from below by raising those forty one by one, until S = 1 / (M (1 + offset)) within 1e-9 S.
    top_p is the upper neighbour of M, so the cut after the first token
    depends on that rounding."""
    rng = np.random.default_rng(seed)
    B = len(offsets)
    bits = np.zeros((B, V), dtype=np.uint16)
    tps = np.zeros(B, dtype=np.float32)
    for b, off in enumerate(offsets):
        x = np.minimum(rng.normal(-9.0, 1.0, V), -6.0)
        x[0] = 0.0
        x[1:41] = -60.0  # the adjustable elements, weight ~1e-26 until set
        rb = W.to_dtype_bits(x, dtype)
        vals = W.bits_to_f32(rb, dtype).astype(np.float64)
        S = float(np.sum(np.exp(vals)))
        # the bf16/fp16 neighbours (b1 < b2) around a target below 1/S
        p_goal = (1.0 / S) * (1.0 - 2.0 ** -5)  # M stays below 1/S: S only grows
        pb = W.bits_to_f32(W.to_dtype_bits(np.array([p_goal]), dtype), dtype)[0]
        b1 = float(pb)
        b2 = float(W.bits_to_f32(W.to_dtype_bits(np.array([pb]), dtype) + np.uint16(1), dtype)[0])
        M = 0.5 * (b1 + b2)
        S_goal = 1.0 / (M * (1.0 + off))
        assert S_goal > S
        j = 1
        while S_goal - S > 1e-9 * S_goal:
            r = S_goal - S
            cand = W.to_dtype_bits(np.array([np.log(r)]), dtype)
            while float(np.exp(np.float64(W.bits_to_f32(cand, dtype)[0]))) > r:
                cand = cand + np.uint16(1)  # one step more negative (sign-magnitude)
            rb[j] = cand[0]
            vals[j] = float(W.bits_to_f32(cand, dtype)[0])
            S = float(np.sum(np.exp(vals)))
            j += 1
            assert j < 41
        rel = (1.0 / S) / M - 1.0
        assert abs(rel - off) < 0.2 * abs(off), (rel, off)
        bits[b] = rb
        tps[b] = np.float32(b2 if top_p_upper else b1)
    return W.Workload(f"near-midpoint {dtype}", dtype, bits, np.ones(B, np.float32), np.zeros(B, np.int32),
                      tps, rng.random(B, dtype=np.float32))

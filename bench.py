#!/usr/bin/env python3
"""Decode-step sampler benchmark on one MI355X.

Workload (default): config C3 -- fp32 logits [256, 128256], per-row
temperature / top-k / top-p mix, one uniform per row (the headline
configuration the metric is quoted on).  A "step" is one mis_sample() call
over the whole batch: the chunk pass (one HBM read of the logits) and the
row pass (per-row finalize); the sampled ids stay on the device.

Inputs are resident in HBM before timing starts.  The batch (131 MB) fits
the 256 MB Infinity Cache, so the timed loop rotates through >= 1 GiB of
distinct copies of it.  Timing uses HIP events on the launch stream:
* whole region (value, ms_per_step): synchronize, start event, K steps with
  nothing else on the streams, end event;
* per step and per pass, in a second run of K steps after it:
  mis_sample_ex() records events before the chunk pass, after it
  on each stream that runs part of it, and after the row pass of every step.
  A batch with fp32 top-p rows and other rows splits the chunk pass into two
  launches on two streams (the top-p rows' on the launch stream, the others'
  on the side stream); both start after the first event, so the chunk pass
  takes from it to the later of the two ends.  That window, which reads every
  row once, is the roofline entry's duration.

The CPU baseline is the literal reference algorithm re-stated with torch CPU
ops (oracle/faithful.py: one call per row, unstable sort, torch.multinomial),
timed on a bounded sample of the same rows, on this host's cores.

Prints one JSON line.

--op attention measures the paged decode attention instead (config A1: a
Llama-3-8B-shaped layer, 32 query / 8 KV heads of 128, block size 16, 64
sequences of 2048 tokens over a 537 MB fp16 pool with scattered blocks, larger
than the Infinity Cache).  A step is one mis_paged_attention() call: the new
K / V written, every head's attention over its sequence.  The roofline entry
covers the call's two launches (the split pass and the merge), whose
algorithmic bytes are the K and V rows read once plus queries, new K / V and
outputs.  The CPU baseline is oracle/attention.py (numpy float64) on a sample
of the sequences.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "rows/sec + HBM GB/s (% of peak), B=256 V=128256 top-k/top-p; p50 µs/step"
WORKLOAD_DESC = {
    "C1": "C1 greedy fp32 [8, 32000]",
    "C2": "C2 stochastic fp16 [8, 32000] T=0.8 k=50 p=0.9",
    "C3": "C3 mixed fp32 [256, 128256] top-k {0,20,1000} / top-p {1,0.95,0.5}, T~U[0.5,1.5]",
    "C4": "C4 single-stream bf16 [1, 152064] top-p 0.95",
    "C5": "C5 edge-stress bf16 [1024, 128256]",
}


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="C3", choices=sorted(WORKLOAD_DESC))
    ap.add_argument("--rotate-gib", type=float, default=1.0, help="distinct input bytes cycled through")
    ap.add_argument("--cpu-rows", type=int, default=32, help="rows in the CPU-baseline sample (0 = skip)")
    ap.add_argument("--cpu-steps", type=int, default=5)
    ap.add_argument("--row-params", default=None, metavar="T,k,p",
                    help="give every row this temperature, top_k and top_p (one row mode at a time, for per-mode "
                         "counters); the default keeps the config's own per-row mix")
    ap.add_argument("--op", default="sample", choices=["sample", "attention", "lmhead"],
                    help="sample: the sampler (configs C1-C5); attention: the paged decode attention (config A1); "
                         "lmhead: the lm_head GEMM fused with the greedy sampler (config L1)")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="after the timed steps, run 5 plain device copies of this many MiB (calibrates "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE against known bytes)")
    return ap.parse_args()


def copy_calibration(mib: int, dev) -> None:
    """Five plain device copies of `mib` MiB (rocprofv3 FETCH_SIZE / WRITE_SIZE calibration)."""
    if mib <= 0:
        return
    import torch
    src = torch.empty(mib << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()


def traffic_from_file(name: str, key: str):
    """HBM bytes per call from a committed rocprofv3 traffic summary under profiles/, or None."""
    try:
        with open(os.path.join(ROOT, "profiles", name)) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def traffic_from_profile(config: str):
    """HBM bytes per chunk pass (its one or two launches of a step) measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    each scaled by the same counter's reading for a copy of known size), from the committed
    summary profiles/k_sample_<config>_traffic.md; None when there is none."""
    path = os.path.join(ROOT, "profiles", f"k_sample_{config}_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_chunk_pass:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def cpu_baseline(w, nrows: int, steps: int) -> dict:
    """Literal reference sampler on the host cores, p50 over `steps` after 2 warmups."""
    import numpy as np
    import torch
    from oracle import faithful

    ncores = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS", ncores) or ncores)
    torch.set_num_threads(max(1, min(ncores, share)))
    B = w.shape[0]
    sel = np.linspace(0, B - 1, min(nrows, B)).round().astype(int)
    sub = w.rows(sel)
    x = sub.to_torch("cpu")
    params = [(float(sub.temperature[i]), int(sub.top_k[i]), float(sub.top_p[i])) for i in range(len(sel))]
    times = []
    torch.manual_seed(0)
    for it in range(2 + steps):
        t0 = time.perf_counter()
        faithful.sample_batch(x, params, literal=True)
        dt = time.perf_counter() - t0
        if it >= 2:
            times.append(dt)
    p50 = statistics.median(times)
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(len(sel) / p50, 2), "unit": "rows/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"{len(sel)} of {B} {w.name} rows (evenly spaced), literal reference algorithm "
                       f"(oracle/faithful.py) one call per row as engine/llm_engine.py:341-344, "
                       f"p50 of {steps} steps after 2 warmups, torch CPU"),
            "p50_ms_per_sample_step": round(p50 * 1e3, 3), "cpu_model": model}


ATT_A1 = {"B": 64, "n_heads": 32, "n_kv_heads": 8, "d_k": 128, "block_size": 16, "context": 2048}


def bench_attention(args):
    """Paged decode attention, config A1 (see the module docstring)."""
    import numpy as np
    import torch
    from vllm_mps_amd import attention as VA

    c = ATT_A1
    B, H, KV, D, bs, ctx = c["B"], c["n_heads"], c["n_kv_heads"], c["d_k"], c["block_size"], c["context"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    mb = ctx // bs
    nb = B * mb + 1
    g = torch.Generator(device="cpu").manual_seed(1)
    pool = torch.randn(nb, 2, bs, KV, D, generator=g).half().to(dev)
    bt = torch.randperm(nb - 1, generator=g)[:B * mb].view(B, mb).int().to(dev)
    sl = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    wi = torch.stack([bt[:, (ctx - 1) // bs], torch.full((B,), (ctx - 1) % bs, dtype=torch.int32, device=dev)],
                     1).int().contiguous()
    q = torch.randn(B, H, D, generator=g).half().to(dev)
    nk = torch.randn(B, KV, D, generator=g).half().to(dev)
    nv = torch.randn(B, KV, D, generator=g).half().to(dev)
    call = lambda: VA.fused_attention_fast(pool, nk, nv, q, bt, sl, wi, H, KV, D, bs)
    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize()
    K = args.steps
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(K):
        call()
    end.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    # per-call durations from events around each call, in a second run
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(K)]
    torch.cuda.synchronize()
    for i in range(K):
        evs[i][0].record()
        call()
        evs[i][1].record()
    torch.cuda.synchronize()
    call_us = [a.elapsed_time(b) * 1e3 for a, b in evs]
    copy_calibration(args.copy_calib_mib, dev)
    mean_us = statistics.mean(call_us)
    kv_bytes = B * ctx * KV * D * 2 * 2
    alg = kv_bytes + B * H * D * 2 * 2 + B * KV * D * 2 * 2   # K/V rows read, queries and outputs, new K/V written
    achieved = alg / (mean_us / 1e6) / 1e9
    res = {
        "metric": "paged decode attention: sequences/s per layer + KV GB/s (% of peak)",
        "value": round(B * K / (total_ms / 1e3), 1),
        "unit": "sequences/s",
        "n_gpus": 1, "steps": K, "warmup": args.warmup,
        "ms_per_step": round(total_ms / K, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 (fp32 arithmetic)", "data": "synthetic",
        "config": {"workload": "A1 Llama-3-8B-shaped decode attention layer, scattered 16-token blocks", **c,
                   "pool_bytes": pool.numel() * 2},
        "p50_us_per_step": round(statistics.median(call_us), 2),
        "roofline": {"bound": "hbm", "kernel": "k_attn_split + k_attn_merge (one call)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_file("paged_attention_A1_traffic.md", "traffic_bytes_per_call"),
                     "algorithmic_bytes_per_launch": alg, "mean_launch_us": round(mean_us, 2)},
    }
    if args.cpu_rows > 0:
        from oracle import attention as A
        ns = min(args.cpu_rows, 8, B)
        sel = np.linspace(0, B - 1, ns).round().astype(int)
        pool_h = pool.cpu().numpy()
        bt_h, sl_h, wi_h = bt.cpu().numpy()[sel], sl.cpu().numpy()[sel], wi.cpu().numpy()[sel]
        q_h, nk_h, nv_h = q.cpu().numpy()[sel], nk.cpu().numpy()[sel], nv.cpu().numpy()[sel]
        from threadpoolctl import threadpool_limits
        times = []
        with threadpool_limits(limits=1):
            for it in range(1 + args.cpu_steps):
                t0 = time.perf_counter()
                A.paged_attention(pool_h, nk_h, nv_h, q_h, bt_h, sl_h, wi_h, H)
                if it >= 1:
                    times.append(time.perf_counter() - t0)
        p50 = statistics.median(times)
        res["cpu_baseline"] = {"value": round(ns / p50, 2), "unit": "sequences/s", "cores": 1, "kind": "port",
                               "sample": f"{ns} of {B} A1 sequences (evenly spaced), oracle/attention.py numpy "
                                         f"float64, p50 of {args.cpu_steps} calls after 1 warmup"}
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


LMH_L1 = {"B": 64, "H": 4096, "V": 128256, "dtype": "bf16"}


def bench_lmhead(args):
    """Fused lm_head + greedy, config L1 (Llama-3-8B's lm_head), against the
    unfused producer + sampler: torch's GEMM in bf16 (hipBLASLt), then
    torch.argmax (the reference's pair) or this build's sampler."""
    import numpy as np
    import torch
    from vllm_mps_amd import lm_head as LH

    c = LMH_L1
    B, H, V = c["B"], c["H"], c["V"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator(device="cpu").manual_seed(1)
    x = (torch.randn(B, H, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    w = (torch.randn(V, H, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    fused = lambda: LH.lm_head_greedy(x, w)
    wt = w.t()
    unfused = lambda: torch.argmax(torch.matmul(x, wt), dim=1)
    # the same GEMM followed by this build's sampler (greedy rows), as an
    # engine without the fusion would run it
    from vllm_mps_amd.sampler import Sampler, pack_params
    smp = Sampler()
    zeros = torch.zeros(B, device=dev)
    packed = pack_params(zeros, torch.zeros(B, dtype=torch.int32, device=dev), torch.ones(B, device=dev), zeros)
    ids_buf = torch.empty(B, dtype=torch.int64, device=dev)
    unfused_mis = lambda: smp.sample_packed(torch.matmul(x, wt), packed, out=ids_buf)
    K = args.steps

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(K):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / K

    # temperature-only rows (T = 1, the default parameters): the fused Gumbel-max
    # draw against the GEMM + this build's sampler with the same rows
    ones = torch.ones(B, device=dev)
    rows_dev = LH.rng_rows((1234, np.arange(B), np.zeros(B, dtype=np.int64)), B, dev)
    fused_t1 = lambda: LH.lm_head_sample(x, w, ones, rows_dev)
    packed_t1 = pack_params(ones, torch.zeros(B, dtype=torch.int32, device=dev), ones, torch.rand(B, device=dev))
    unfused_t1 = lambda: smp.sample_packed(torch.matmul(x, wt), packed_t1, out=ids_buf)
    # every pipeline twice, round robin; the second round is reported (the
    # first one also brings the clocks up to speed for the pipeline timed first)
    for _ in range(2):
        ms, ms_unfused, ms_unfused_mis, ms_t1, ms_unfused_t1 = (
            timed(f) for f in (fused, unfused, unfused_mis, fused_t1, unfused_t1))
    same = bool(torch.equal(fused(), unfused())) and bool(torch.equal(fused(), unfused_mis().clone()))
    copy_calibration(args.copy_calib_mib, dev)
    alg = V * H * 2 + B * H * 2 + B * 8           # the weight read once, the hidden states, the ids
    achieved = alg / (ms / 1e3) / 1e9
    flops = 2.0 * B * H * V
    res = {
        "metric": "fused lm_head + greedy: sequences/s per decode step + weight GB/s (% of peak)",
        "value": round(B / (ms / 1e3), 1), "unit": "sequences/s",
        "n_gpus": 1, "steps": K, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 (fp32 accumulation)", "data": "synthetic",
        "config": {"workload": "L1 Llama-3-8B lm_head [4096 -> 128256] bf16, greedy", **c},
        "unfused_ms_per_step": round(ms_unfused, 5),
        "speedup_vs_unfused": round(ms_unfused / ms, 3),
        "unfused_mis_sampler_ms_per_step": round(ms_unfused_mis, 5),
        "speedup_vs_unfused_mis_sampler": round(ms_unfused_mis / ms, 3),
        "temperature_rows": {"fused_ms_per_step": round(ms_t1, 5), "unfused_mis_sampler_ms_per_step": round(ms_unfused_t1, 5),
                             "speedup": round(ms_unfused_t1 / ms_t1, 3)},
        "ids_equal_unfused": same,
        "tflops": round(flops / (ms / 1e3) / 1e12, 1),
        "roofline": {"bound": "hbm", "kernel": "k_lmh_tile + k_lmh_merge (one call)", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_file("lm_head_greedy_L1_traffic.md", "traffic_bytes_per_call"),
                     "algorithmic_bytes_per_launch": alg, "mean_launch_us": round(ms * 1e3, 2)},
    }
    if args.cpu_rows > 0:
        from oracle import lm_head as O
        from threadpoolctl import threadpool_limits
        ns = 2
        xs = x[:ns].float().cpu().numpy()
        ws = w.float().cpu().numpy()
        times = []
        with threadpool_limits(limits=1):
            for it in range(1 + min(args.cpu_steps, 3)):
                t0 = time.perf_counter()
                O.greedy(xs, ws, "bf16")
                if it >= 1:
                    times.append(time.perf_counter() - t0)
        p50 = statistics.median(times)
        res["cpu_baseline"] = {"value": round(ns / p50, 3), "unit": "sequences/s", "cores": 1, "kind": "port",
                               "sample": f"{ns} of {B} L1 sequences, oracle/lm_head.py numpy float64 GEMM + argmax, "
                                         f"p50 of {len(times)} calls after 1 warmup"}
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "rows are independent, so N GPUs would each run this single-GPU step on B/N rows.",
              file=sys.stderr)
        sys.exit(2)
    if args.op == "attention":
        bench_attention(args)
        return
    if args.op == "lmhead":
        bench_lmhead(args)
        return

    import torch
    from vllm_mps_amd import workloads as W
    from vllm_mps_amd.sampler import Sampler, pack_params, row_kinds

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    w = W.make(args.config)
    B, V = w.shape
    if args.row_params:
        import numpy as np
        t_, k_, p_ = args.row_params.split(",")
        w = W.Workload(w.name, w.dtype, w.logits, np.full(B, float(t_), np.float32), np.full(B, int(k_), np.int32),
                       np.full(B, float(p_), np.float32), w.uniform)
    esz = 4 if w.dtype == "f32" else 2
    bytes_alg = W.algorithmic_bytes(B, V, w.dtype)
    nbuf = max(1, math.ceil(args.rotate_gib * (1 << 30) / (B * V * esz)))
    base = w.to_torch(dev)
    base_dtype = base.dtype
    bufs = [base.clone() for _ in range(nbuf)]
    del base
    packed = pack_params(torch.from_numpy(w.temperature.copy()).to(dev), torch.from_numpy(w.top_k.copy()).to(dev),
                         torch.from_numpy(w.top_p.copy()).to(dev), torch.from_numpy(w.uniform.copy()).to(dev))
    out = torch.empty(B, dtype=torch.int64, device=dev)
    # the engine knows its requests' parameters on the host: the row-kind hint
    kinds = row_kinds(w.temperature, w.top_k, w.top_p, V, base_dtype)
    s = Sampler()
    for i in range(args.warmup):
        s.sample_packed(bufs[i % nbuf], packed, out=out, kinds=kinds)
    torch.cuda.synchronize()

    K = args.steps
    # the timed region: K steps with nothing else on the streams
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(K):
        s.sample_packed(bufs[(args.warmup + i) % nbuf], packed, out=out, kinds=kinds)
    end.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    # then K more steps with events inside each, for the per-step and per-pass
    # durations (the events themselves cost about 13 us per C3 step, so they
    # stay out of the timed region)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(K)]
    for trio in evs:
        for e in trio:
            e.record()
    torch.cuda.synchronize()
    for i in range(K):
        s.sample_packed(bufs[(args.warmup + K + i) % nbuf], packed, out=out, events=evs[i], kinds=kinds)
    torch.cuda.synchronize()
    step_us = [t[0].elapsed_time(t[2]) * 1e3 for t in evs]
    # the chunk pass: from the first event to the later end of its launches
    # (two, and the fourth event recorded, exactly for fp32 with both kinds)
    split = w.dtype == "f32" and (kinds & 3) == 3
    k1_us = [(max(t[0].elapsed_time(t[1]), t[0].elapsed_time(t[3])) if split else t[0].elapsed_time(t[1])) * 1e3
             for t in evs]
    k2_us = [st - k1 for st, k1 in zip(step_us, k1_us)]  # the rest of the step
    ms_per_step = total_ms / K
    rows_per_s = B * K / (total_ms / 1e3)
    gbs_step = bytes_alg / (ms_per_step / 1e3) / 1e9
    k1_mean, k2_mean = statistics.mean(k1_us), statistics.mean(k2_us)
    bytes_k1 = B * V * esz + 16 * B  # logits + params: the chunk pass's HBM read
    # the roofline entry is the chunk pass's: the pass that moves the
    # algorithmic bytes (one launch, or two on two streams inside one window)
    # and the longest.  The row pass is up to seven shorter launches on two
    # streams whose algorithmic bytes are only the ids (their re-reads of rows
    # are not algorithmic); its time is reported beside it.
    dom, dom_us, dom_bytes = "k_sample", k1_mean, bytes_k1
    q = statistics.quantiles(step_us, n=10)
    achieved = dom_bytes / (dom_us / 1e6) / 1e9
    res = {
        "metric": METRIC,
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": "synthetic",
        "config": {"workload": WORKLOAD_DESC[args.config], "B": B, "V": V, "seed": W.SEEDS[args.config],
                   "rotating_buffers": nbuf, "rotated_bytes": nbuf * B * V * esz,
                   **({"row_params": args.row_params} if args.row_params else {})},
        "tokens_per_s": round(rows_per_s, 1),
        "p50_us_per_step": round(statistics.median(step_us), 2),
        "p90_us_per_step": round(q[8], 2),
        "hbm_gbs_step": round(gbs_step, 1),
        "hbm_frac_step": round(gbs_step / HBM_PEAK_GBS, 4),
        "algorithmic_bytes_per_step": bytes_alg,
        "kernels_us": {"k_sample": round(k1_mean, 2), "row_pass": round(k2_mean, 2)},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profile(args.config) if dom == "k_sample" else None,
                     "algorithmic_bytes_per_launch": dom_bytes, "mean_launch_us": round(dom_us, 2),
                     "chunk_pass_launches": 2 if split else 1,
                     "row_pass_us": round(k2_mean, 2)},
    }
    copy_calibration(args.copy_calib_mib, dev)
    if args.cpu_rows > 0:
        res["cpu_baseline"] = cpu_baseline(w, args.cpu_rows, args.cpu_steps)
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()

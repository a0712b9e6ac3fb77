"""Seeded synthetic decode-step workloads (the five sampler configurations).

Every workload is a ``[B, V]`` logits batch plus per-row sampling parameters
and one uniform per row.  Generation is pure numpy (PCG64 ``default_rng``), so
the same seed gives the same bytes on every machine with this numpy; tests
pin that with SHA-256 digests.  Values are drawn in float64, rounded to
float32 (RNE) and then to the 16-bit dtype (RNE) where one is used.  16-bit
logits are carried as ``uint16`` bit patterns.

Configs (shapes and mixes of the reference's engine: ``config.py:18,27``
gives B=8, V=32000; ``run_demo.py:48`` / ``examples/basic_generation.py:55``
give T=0.8, top_p=0.9):

* C1  greedy fp32 [8, 32000], N(0, 3^2), T=0.
* C2  stochastic fp16 [8, 32000], N(0, 3^2) + one +8 spike per row,
      T=0.8, top_k=50, top_p=0.9.
* C3  mixed fp32 [256, 128256]: 64 near-one-hot rows (N(0,1) + 20 at one
      index), 128 N(0, 3^2) rows, 64 Zipf rows (-1.1 ln(rank) under a
      permutation); T ~ U[0.5, 1.5], top_k in {0, 20, 1000},
      top_p in {1.0, 0.95, 0.5} per row.
* C4  single stream bf16 [1, 152064], N(0, 2.5^2) + 64 distinct +6 spikes,
      T=1, top_k off, top_p=0.95.
* C5  edge stress bf16 [1024, 128256], N(0, 3^2) with round(0.1 V) -inf
      entries per row, 51 rows holding an exact duplicate of the row max;
      param classes {T=0}, {T=1,k=V}, {T=1,k=1}, {T=1,p=0.01},
      {T=1,k=V,p=0.01}, each class holding at least one duplicate-max row.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np

SEEDS = {"C1": 1001, "C2": 1002, "C3": 1003, "C4": 1004, "C5": 1005}
UNIFORM_SEED_OFFSET = 1_000_000
SHAPES = {"C1": (8, 32000, "f32"), "C2": (8, 32000, "f16"), "C3": (256, 128256, "f32"),
          "C4": (1, 152064, "bf16"), "C5": (1024, 128256, "bf16")}


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (RNE; NaN stays NaN) -> uint16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u.astype(np.uint64) + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_dtype_bits(x64: np.ndarray, dtype: str) -> np.ndarray:
    x32 = np.asarray(x64, dtype=np.float64).astype(np.float32)
    if dtype == "f32":
        return x32
    if dtype == "f16":
        return x32.astype(np.float16).view(np.uint16)
    return f32_to_bf16_bits(x32)


def bits_to_f32(raw: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "f32":
        return raw.astype(np.float32, copy=False)
    if dtype == "f16":
        return raw.view(np.float16).astype(np.float32)
    return bf16_bits_to_f32(raw)


@dataclass
class Workload:
    name: str
    dtype: str              # "f32" | "f16" | "bf16"
    logits: np.ndarray      # [B, V] float32, or uint16 bit patterns for 16-bit
    temperature: np.ndarray  # [B] float32
    top_k: np.ndarray       # [B] int32
    top_p: np.ndarray       # [B] float32 (already the f32 threshold)
    uniform: np.ndarray     # [B] float32 in [0, 1)

    @property
    def shape(self):
        return self.logits.shape

    def digest(self) -> str:
        h = hashlib.sha256()
        h.update(np.ascontiguousarray(self.logits).tobytes())
        for a in (self.temperature, self.top_k, self.top_p, self.uniform):
            h.update(np.ascontiguousarray(a).tobytes())
        return h.hexdigest()

    def rows(self, sel) -> "Workload":
        return Workload(self.name, self.dtype, np.ascontiguousarray(self.logits[sel]),
                        self.temperature[sel].copy(), self.top_k[sel].copy(),
                        self.top_p[sel].copy(), self.uniform[sel].copy())

    def to_torch(self, device="cpu"):
        """Logits as a torch tensor of the workload dtype on ``device``."""
        import torch
        if self.dtype == "f32":
            t = torch.from_numpy(np.ascontiguousarray(self.logits))
        elif self.dtype == "f16":
            t = torch.from_numpy(np.ascontiguousarray(self.logits).view(np.float16))
        else:
            t = torch.from_numpy(np.ascontiguousarray(self.logits).view(np.int16)).view(torch.bfloat16)
        return t.to(device)


def _uniforms(seed: int, B: int) -> np.ndarray:
    return np.random.default_rng(seed + UNIFORM_SEED_OFFSET).random(B, dtype=np.float32)


def make_c1() -> Workload:
    B, V, dt = SHAPES["C1"]
    rng = np.random.default_rng(SEEDS["C1"])
    x = to_dtype_bits(rng.normal(0.0, 3.0, (B, V)), dt)
    return Workload("C1", dt, x, np.zeros(B, np.float32), np.zeros(B, np.int32),
                    np.ones(B, np.float32), _uniforms(SEEDS["C1"], B))


def make_c2() -> Workload:
    B, V, dt = SHAPES["C2"]
    rng = np.random.default_rng(SEEDS["C2"])
    x = rng.normal(0.0, 3.0, (B, V))
    spike = rng.integers(0, V, B)
    x[np.arange(B), spike] += 8.0
    return Workload("C2", dt, to_dtype_bits(x, dt), np.full(B, 0.8, np.float32),
                    np.full(B, 50, np.int32), np.full(B, 0.9, np.float32), _uniforms(SEEDS["C2"], B))


def make_c3() -> Workload:
    B, V, dt = SHAPES["C3"]
    rng = np.random.default_rng(SEEDS["C3"])
    T = rng.uniform(0.5, 1.5, B).astype(np.float32)
    k = rng.choice(np.array([0, 20, 1000], np.int32), B)
    p = rng.choice(np.array([1.0, 0.95, 0.5], np.float32), B)
    kinds = rng.permutation(np.array([0] * 64 + [1] * 128 + [2] * 64))
    x = np.empty((B, V), np.float32)
    for b in range(B):
        if kinds[b] == 0:
            row = rng.normal(0.0, 1.0, V)
            row[rng.integers(0, V)] += 20.0
        elif kinds[b] == 1:
            row = rng.normal(0.0, 3.0, V)
        else:
            ranks = rng.permutation(V) + 1
            row = -1.1 * np.log(ranks.astype(np.float64))
        x[b] = row.astype(np.float32)
    return Workload("C3", dt, x, T, k.astype(np.int32), p.astype(np.float32), _uniforms(SEEDS["C3"], B))


def c3_row_kinds() -> np.ndarray:
    """0 near-one-hot, 1 gaussian, 2 zipf -- the C3 row mix, same draws as make_c3."""
    B = SHAPES["C3"][0]
    rng = np.random.default_rng(SEEDS["C3"])
    rng.uniform(0.5, 1.5, B)
    rng.choice(np.array([0, 20, 1000], np.int32), B)
    rng.choice(np.array([1.0, 0.95, 0.5], np.float32), B)
    return rng.permutation(np.array([0] * 64 + [1] * 128 + [2] * 64))


def make_c4() -> Workload:
    B, V, dt = SHAPES["C4"]
    rng = np.random.default_rng(SEEDS["C4"])
    x = rng.normal(0.0, 2.5, (B, V))
    spikes = rng.choice(V, 64, replace=False)
    x[0, spikes] += 6.0
    return Workload("C4", dt, to_dtype_bits(x, dt), np.ones(B, np.float32), np.zeros(B, np.int32),
                    np.full(B, 0.95, np.float32), _uniforms(SEEDS["C4"], B))


C5_CLASSES = [  # (temperature, top_k or -1 for V, top_p)
    (0.0, 0, 1.0),
    (1.0, -1, 1.0),
    (1.0, 1, 1.0),
    (1.0, 0, 0.01),
    (1.0, -1, 0.01),
]


def make_c5(rows: int | None = None) -> Workload:
    """C5; ``rows`` limits generation to the first rows (same bytes as the full batch's prefix)."""
    B, V, dt = SHAPES["C5"]
    rng = np.random.default_rng(SEEDS["C5"])
    cls = rng.integers(0, len(C5_CLASSES), B)
    dup = []
    for c in range(len(C5_CLASSES)):
        members = np.nonzero(cls == c)[0]
        dup.append(int(rng.choice(members)))
    rest = np.setdiff1d(np.arange(B), np.array(dup))
    dup.extend(int(v) for v in rng.choice(rest, 51 - len(dup), replace=False))
    dup_set = set(dup)
    n_inf = int(round(0.1 * V))
    T = np.array([C5_CLASSES[c][0] for c in cls], np.float32)
    k = np.array([V if C5_CLASSES[c][1] < 0 else C5_CLASSES[c][1] for c in cls], np.int32)
    p = np.array([C5_CLASSES[c][2] for c in cls], np.float32)
    u = _uniforms(SEEDS["C5"], B)
    nb = B if rows is None else rows
    x = np.empty((nb, V), np.uint16)
    for b in range(nb):
        row = rng.normal(0.0, 3.0, V)
        row[rng.choice(V, n_inf, replace=False)] = -np.inf
        bits = to_dtype_bits(row, dt)
        if b in dup_set:
            vals = bf16_bits_to_f32(bits)
            amax = int(np.argmax(vals))
            finite = np.nonzero(np.isfinite(vals))[0]
            finite = finite[finite != amax]
            j = int(finite[rng.integers(0, finite.shape[0])])
            bits[j] = bits[amax]
        x[b] = bits
    w = Workload("C5", dt, x, T, k, p, u)
    return w if rows is None else w.rows(slice(0, rows))


def c5_row_classes() -> np.ndarray:
    """Index into C5_CLASSES of every C5 row (same draws as make_c5)."""
    rng = np.random.default_rng(SEEDS["C5"])
    return rng.integers(0, len(C5_CLASSES), SHAPES["C5"][0])


def c5_duplicate_rows() -> list[int]:
    """Rows of C5 holding an exact duplicate maximum (same draws as make_c5)."""
    B = SHAPES["C5"][0]
    rng = np.random.default_rng(SEEDS["C5"])
    cls = rng.integers(0, len(C5_CLASSES), B)
    dup = [int(rng.choice(np.nonzero(cls == c)[0])) for c in range(len(C5_CLASSES))]
    rest = np.setdiff1d(np.arange(B), np.array(dup))
    dup.extend(int(v) for v in rng.choice(rest, 51 - len(dup), replace=False))
    return sorted(dup)


MAKERS = {"C1": make_c1, "C2": make_c2, "C3": make_c3, "C4": make_c4, "C5": make_c5}


def make(name: str) -> Workload:
    return MAKERS[name]()


def algorithmic_bytes(B: int, V: int, dtype: str) -> int:
    """One read of every logits row + 16 B of params/uniform in + 8 B id out per row."""
    esz = 4 if dtype == "f32" else 2
    return B * V * esz + 24 * B

"""GPU-vs-oracle comparison (test infrastructure only).

The bar, per row with status OK in both:
* status: identical.
* keep mask: bit-exact.  The one exemption is an fp32 top-p row whose oracle
  decision margin |E - f32(top_p)| at the cut is below TOPP_MARGIN (the GPU
  sums float64 masses, the oracle x87 long double); such rows are reported.
* token id: identical unless the uniform lies within DRAW_MARGIN (relative to
  the kept mass) of a CDF edge, or the row's mask was exempted.  A
  temperature-only row (T > 0, top-k off, top_p = 1) draws from weights the
  GPU computes in float32 with a relative error of at most 4.8e-7 each (wexp);
  its margin is TEMP_DRAW_MARGIN.
* post-filter probabilities: within 1e-5 relative (fp32) or 2e-3 relative
  (fp16/bf16) of the oracle's, on the kept set; exactly 0 elsewhere.
Greedy rows: identical ids.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

TOPP_MARGIN = 1e-12
DRAW_MARGIN = 1e-9
TEMP_DRAW_MARGIN = 1e-6  # above 2 x 4.8e-7: every weight's error, and so the CDF's, is below that share
PROB_RTOL = {"f32": 1e-5, "f16": 2e-3, "bf16": 2e-3}
# two ulps of the dtype's smallest subnormal: below the normal range the
# conversion of a probability to the dtype keeps only a few significant bits
PROB_ATOL = {"f32": 2.0 ** -148, "f16": 2.0 ** -23, "bf16": 2.0 ** -132}


@dataclass
class Report:
    rows: int = 0
    ok: bool = True
    failures: list = field(default_factory=list)
    exempt_mask: list = field(default_factory=list)
    exempt_draw: list = field(default_factory=list)

    def fail(self, msg):
        self.ok = False
        self.failures.append(msg)

    def summary(self) -> str:
        return (f"rows={self.rows} ok={self.ok} failures={len(self.failures)} "
                f"mask-exempt={len(self.exempt_mask)} draw-exempt={len(self.exempt_draw)}"
                + ("" if self.ok else "\n  " + "\n  ".join(self.failures[:20])))


def unpack_keep(words: np.ndarray, V: int) -> np.ndarray:
    """[B, ceil(V/32)] uint32/int32 bitmask -> [B, V] bool (bit j%32 of word j/32)."""
    w = np.ascontiguousarray(words).view(np.uint32)
    bits = np.unpackbits(w.view(np.uint8).reshape(w.shape[0], -1, 4)[:, :, ::-1], axis=2)
    bits = bits[:, :, ::-1].reshape(w.shape[0], -1)  # little-endian bit order per word
    return bits[:, :V].astype(bool)


def compare(dtype: str, params: np.ndarray, gpu: dict, orc: dict) -> Report:
    """gpu: ids [B], status [B], and optionally keep [B,V] bool, probs [B,V]."""
    rep = Report(rows=int(orc["ids"].shape[0]))
    B = rep.rows
    for b in range(B):
        so, sg = int(orc["status"][b]), int(gpu["status"][b])
        if so != sg:
            rep.fail(f"row {b}: status gpu={sg} oracle={so}")
            continue
        if so != 0:
            if int(gpu["ids"][b]) != -1:
                rep.fail(f"row {b}: id {int(gpu['ids'][b])} for a row with status {so}")
            continue
        T = float(params["temperature"][b])
        mask_exempt = False
        if "keep" in gpu and "keep" in orc:
            kg, ko = gpu["keep"][b], orc["keep"][b]
            if not np.array_equal(kg, ko):
                ndiff = int((kg != ko).sum())
                tm = float(orc["topp_margin"][b])
                if dtype == "f32" and params["top_p"][b] < 1.0 and T != 0.0 and np.isfinite(tm) and tm < TOPP_MARGIN:
                    rep.exempt_mask.append((b, ndiff, tm))
                    mask_exempt = True
                else:
                    first = int(np.nonzero(kg != ko)[0][0])
                    rep.fail(f"row {b}: keep mask differs in {ndiff} places (first j={first} gpu={bool(kg[first])}); "
                             f"n_kept oracle={int(orc['n_kept'][b])} gpu={int(kg.sum())} topp_margin={tm:.3g}")
                    continue
        ig, io = int(gpu["ids"][b]), int(orc["ids"][b])
        if ig != io:
            dm = float(orc["draw_margin"][b])
            V = orc["probs"].shape[1] if "probs" in orc else None
            k = int(params["top_k"][b])
            temp_only = T > 0.0 and (k == 0 or (V is not None and k >= V)) and float(params["top_p"][b]) >= 1.0
            margin = TEMP_DRAW_MARGIN if temp_only else DRAW_MARGIN
            if T != 0.0 and (mask_exempt or (np.isfinite(dm) and dm < margin)):
                rep.exempt_draw.append((b, ig, io, dm))
            else:
                rep.fail(f"row {b}: id gpu={ig} oracle={io} draw_margin={dm:.3g}")
                continue
        if "probs" in gpu and "probs" in orc and not mask_exempt:
            pg, po = gpu["probs"][b].astype(np.float64), orc["probs"][b].astype(np.float64)
            # subnormal results carry less relative precision than the dtype's
            # normal range: the error may reach PROB_ATOL (two subnormal ulps)
            atol = PROB_ATOL[dtype]
            z = po == 0.0
            if np.any(np.abs(pg[z]) > atol):
                rep.fail(f"row {b}: nonzero prob where the oracle has 0")
                continue
            nz = ~z
            if np.any(nz):
                err = np.abs(pg[nz] - po[nz])
                bad = err > np.maximum(PROB_RTOL[dtype] * po[nz], atol)
                if np.any(bad):
                    rel = err / po[nz]
                    k = int(np.argmax(np.where(bad, rel, -1.0)))
                    j = int(np.nonzero(nz)[0][k])
                    rep.fail(f"row {b}: prob rel err {rel[k]:.3g} at j={j} gpu={pg[j]} oracle={po[j]}")
    return rep

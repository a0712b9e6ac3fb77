"""Writes tests/golden/c3_fp32_topp_deviation.json (run from the repo root).

Every C3 row with top-p active (top_p < 1) where the build's fp32 top-p
contract (exact softmax masses, oracle/mis_oracle.c) keeps a different set
than the reference's own op sequence run in torch fp32 (model/sampler.py:
46-55: float softmax, cumsum, exclusive mass, ``>= top_p``; contract mode:
stable sort), with the oracle's decision margin |E - f32(top_p)| at the cut.
Computed with the installed torch on this host (torch 2.10, x86-64 CPU); the
reference itself is not imported.
"""
from __future__ import annotations

import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402
import torch  # noqa: E402

from oracle import faithful  # noqa: E402
from oracle import oracle as O  # noqa: E402
from tests import harness as H  # noqa: E402
from vllm_mps_amd import workloads as W  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c3_fp32_topp_deviation.json")


def deviations():
    w = W.make_c3()
    r = O.sample_rows(w.logits, "f32", H.params_of(w), want_keep=True)
    t = torch.from_numpy(np.ascontiguousarray(w.logits))
    rows = []
    for b in range(w.shape[0]):
        T, k, p = float(w.temperature[b]), int(w.top_k[b]), float(w.top_p[b])
        if not (p < 1.0):
            continue
        _, probs = faithful.row_sample(t[b], T, k, p, uniform=0.5, literal=False, return_probs=True)
        keep_t = (probs > 0).numpy()
        keep_o = r["keep"][b]
        if not np.array_equal(keep_t, keep_o):
            rows.append(dict(row=b, top_k=k, top_p=p, temperature=T, n_kept_oracle=int(keep_o.sum()),
                             n_kept_torch=int(keep_t.sum()), margin=float(r["topp_margin"][b])))
    n_topp = int((w.top_p < 1.0).sum())
    return n_topp, rows


if __name__ == "__main__":
    n, rows = deviations()
    with open(OUT, "w") as f:
        json.dump(dict(config="C3", topp_rows=n, torch=torch.__version__, rows=rows), f, indent=1)
    print(f"{len(rows)} of {n} top-p rows differ; margins {[round(x['margin'], 12) for x in rows]}")

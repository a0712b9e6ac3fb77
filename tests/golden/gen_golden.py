"""Write the golden fixtures for the sampler configurations.

The reference (vllm_mps) ships no sampler tests, fixtures or golden vectors
(its only pinned behaviour on this boundary is SamplingParams validation,
tests/test_sequence.py:55-64), so these fixtures are produced by the CPU
oracle -- which tests/test_oracle_pin.py pins independently against torch,
numpy and exact arithmetic -- and serve as regression pins:

* digests.json     SHA-256 of every generated workload (logits + params).
* c1_c2.npz        C1 and C2 in full: ids, status, keep masks (packed bits),
                   kept indices and post-filter probabilities.
* rows.json        per-row summaries for C3 (256 rows), C4 and C5 (1024
                   rows): id, status, kept count, cut value / index, keep-mask
                   SHA-1, top-p and draw margins.

Run from the repo root:  python tests/golden/gen_golden.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from vllm_mps_amd import workloads as W  # noqa: E402


def params_of(w):
    return O.make_params(w.temperature, w.top_k, w.top_p, w.uniform)


def mask_sha1(keep_row: np.ndarray) -> str:
    return hashlib.sha1(np.packbits(keep_row.astype(np.uint8)).tobytes()).hexdigest()


def row_summaries(w, res) -> list[dict]:
    out = []
    for b in range(w.shape[0]):
        out.append({
            "id": int(res["ids"][b]), "status": int(res["status"][b]), "n_kept": int(res["n_kept"][b]),
            "cut_value": float(res["cut_value"][b]) if np.isfinite(res["cut_value"][b]) else None,
            "cut_index": int(res["cut_index"][b]), "keep_sha1": mask_sha1(res["keep"][b]),
            "topp_margin": None if not np.isfinite(res["topp_margin"][b]) else float(res["topp_margin"][b]),
            "draw_margin": None if not np.isfinite(res["draw_margin"][b]) else float(res["draw_margin"][b]),
        })
    return out


def main():
    digests, rows = {}, {}
    npz = {}
    for name in ["C1", "C2", "C3", "C4", "C5"]:
        w = W.make(name)
        digests[name] = w.digest()
        res = O.sample_rows(w.logits, w.dtype, params_of(w), want_probs=(name in ("C1", "C2")), want_keep=True)
        if name in ("C1", "C2"):
            keep = res["keep"]
            npz[f"{name}_ids"] = res["ids"]
            npz[f"{name}_status"] = res["status"]
            npz[f"{name}_keep_bits"] = np.packbits(keep.astype(np.uint8), axis=1)
            kept_idx = np.nonzero(keep)
            npz[f"{name}_kept_rows"] = kept_idx[0].astype(np.int32)
            npz[f"{name}_kept_cols"] = kept_idx[1].astype(np.int32)
            npz[f"{name}_kept_probs"] = res["probs"][kept_idx].astype(np.float32)
        else:
            rows[name] = row_summaries(w, res)
        print(name, w.shape, digests[name][:16], flush=True)
    with open(os.path.join(HERE, "digests.json"), "w") as f:
        json.dump(digests, f, indent=1, sort_keys=True)
    with open(os.path.join(HERE, "rows.json"), "w") as f:
        json.dump(rows, f, separators=(",", ":"))
    np.savez_compressed(os.path.join(HERE, "c1_c2.npz"), **npz)


if __name__ == "__main__":
    main()

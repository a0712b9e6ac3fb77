"""The reference sampler's algorithm re-stated with torch CPU ops.

TEST INFRASTRUCTURE / CPU BASELINE ONLY (see ``oracle/__init__.py``).

``row_sample`` performs, per row, the op sequence of ``model/sampler.py:28-60``:
true division by the temperature (:37), ``topk`` + ``where`` (:40-43), sort,
softmax, cumsum, exclusive-mass mask and scatter (:46-55), and a final
softmax + draw (:58-60).  Two switches select between:

* ``literal=True`` -- the reference as written: unstable ``torch.sort`` and
  ``torch.multinomial`` from the global generator.  This is the CPU
  throughput baseline, run one row per call exactly as
  ``engine/llm_engine.py:341-344`` does.
* ``literal=False`` -- the same ops under the build's contract: a stable sort
  (ties -> lowest index) and an inverse-CDF draw from a caller-supplied
  uniform.  For fp16/bf16 this reproduces torch's own rounding chain, so the
  tests use it to pin the C oracle's 16-bit chain against torch itself.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def row_sample(logits: torch.Tensor, temperature: float, top_k: int, top_p: float,
               uniform: float | None = None, literal: bool = True, return_probs: bool = False):
    if temperature == 0.0:
        tok = int(torch.argmax(logits).item())
        return (tok, None) if return_probs else tok
    z = logits / temperature
    if top_k > 0:
        kk = min(top_k, z.shape[-1])
        kth = torch.topk(z, kk).values[-1]
        z = torch.where(z < kth, torch.full_like(z, float("-inf")), z)
    if top_p < 1.0:
        order_vals, order_idx = torch.sort(z, descending=True, stable=not literal)
        p_sorted = F.softmax(order_vals, dim=-1)
        exclusive = torch.cumsum(p_sorted, dim=-1) - p_sorted
        order_vals = order_vals.masked_fill(exclusive >= top_p, float("-inf"))
        z = torch.empty_like(z).scatter_(-1, order_idx, order_vals)
    probs = F.softmax(z, dim=-1)
    if literal:
        tok = int(torch.multinomial(probs, num_samples=1).item())
    else:
        w = probs.double()
        cdf = torch.cumsum(w, dim=-1)
        target = float(uniform) * float(cdf[-1])
        hits = torch.nonzero(cdf > target)
        tok = int(hits[0].item()) if hits.numel() else int(torch.nonzero(w > 0)[-1].item())
    return (tok, probs) if return_probs else tok


def sample_batch(logits: torch.Tensor, params, uniforms=None, literal: bool = True) -> list[int]:
    """One call per row with that row's params -- the engine's call pattern."""
    out = []
    for i in range(logits.shape[0]):
        t, k, p = params[i]
        u = None if uniforms is None else float(uniforms[i])
        out.append(row_sample(logits[i], t, k, p, u, literal=literal))
    return out

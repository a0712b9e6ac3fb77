"""The engine's per-step sampling as one batched call.

The reference engine samples each running sequence on its own
(``engine/llm_engine.py:339-345``, ``_step_adapter``)::

    for i, seq_id in enumerate(seq_ids):
        params = self._seq_to_params.get(seq_id, SamplingParams())
        token = self.sampler.sample(logits[i], params)

one Python call, one ``torch.multinomial`` and one ``.item()`` host
synchronisation per row.  ``StepSampler.sample_step`` takes the same inputs
(the step's ``[B, V]`` logits, the sequence ids in row order, the engine's
``_seq_to_params`` map) and returns the same ``list[int]``, from one launch
sequence over the whole batch and a single device-to-host copy of ids and
row statuses.

Each row's uniform comes from the per-request device generator keyed by
(``seed``, request = sequence id, step = tokens this object has sampled for
that sequence), so a sequence's token depends on its own logits and history
only, not on which other sequences share the batch or in what order.
``release(seq_id)`` forgets a finished sequence's step counter (the engine
evicts a finished sequence's state in ``_update_sequences``,
``engine/llm_engine.py:366-371``).

Errors surface as the reference's do: a row the library rejects raises
``ValueError`` (invalid parameters, ``core/sequence.py:41-61``) or
``RuntimeError`` (invalid distribution, ``torch.multinomial`` at
``model/sampler.py:59``), for the first such row in batch order, and no step
counter advances.
"""
from __future__ import annotations

from typing import Mapping, Sequence

import numpy as np
import torch

from . import _native
from .sampler import Sampler
from .sampling_params import SamplingParams


class StepSampler:
    """Batched replacement of the engine's per-row sampling loop."""

    def __init__(self, seed: int = 0, sampler: Sampler | None = None) -> None:
        if not 0 <= int(seed) < 1 << 64:
            raise ValueError("seed must lie in [0, 2^64)")
        self.seed = int(seed)
        self.sampler = Sampler() if sampler is None else sampler
        self._steps: dict[int, int] = {}
        self._dev: dict[int, torch.Tensor] = {}   # device: ids (int64) then statuses (int32)
        self._host: torch.Tensor | None = None    # pinned staging of the same bytes

    def step_of(self, seq_id: int) -> int:
        """Draws taken so far for ``seq_id`` (the next draw's step)."""
        return self._steps.get(seq_id, 0)

    def release(self, seq_id: int) -> None:
        """Forget a finished sequence's step counter."""
        self._steps.pop(seq_id, None)

    def _buffers(self, dev: torch.device, B: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        idx = dev.index if dev.index is not None else torch.cuda.current_device()
        nbytes = 12 * B
        buf = self._dev.get(idx)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
            self._dev[idx] = buf
        if self._host is None or self._host.numel() < nbytes:
            self._host = torch.empty(max(nbytes, 256), dtype=torch.uint8, pin_memory=True)
        ids = buf[:8 * B].view(torch.int64)
        status = buf[8 * B:12 * B].view(torch.int32)
        return buf[:nbytes], ids, status

    def sample_step(self, logits: torch.Tensor, seq_ids: Sequence[int],
                    seq_to_params: Mapping[int, SamplingParams]) -> list[int]:
        """Next token of every row: ``logits[i]`` belongs to ``seq_ids[i]``,
        whose parameters are ``seq_to_params.get(seq_id, SamplingParams())``
        as in the reference loop."""
        if logits.dim() != 2 or logits.shape[0] != len(seq_ids):
            raise ValueError(f"logits {tuple(logits.shape)} do not match {len(seq_ids)} sequence ids")
        B = len(seq_ids)
        if B == 0:
            return []
        if len(set(seq_ids)) != B:
            raise ValueError("a sequence id appears twice in one step")
        params = [seq_to_params.get(s, SamplingParams()) for s in seq_ids]
        steps = [self._steps.get(s, 0) for s in seq_ids]
        dev = logits.device
        both, ids, status = self._buffers(dev, B)
        self.sampler.sample_rows(logits, params, rng=(self.seed, list(seq_ids), steps), out=ids, status_out=status)
        host = self._host[:12 * B]
        host.copy_(both, non_blocking=True)
        torch.cuda.current_stream(dev).synchronize()
        raw = host.numpy()
        hid = raw[:8 * B].view(np.int64)
        hst = raw[8 * B:].view(np.int32)
        for s in hst:
            if s != _native.ROW_OK:
                # raises ValueError / RuntimeError as the reference would
                self.sampler._checked(torch.from_numpy(hid.copy()), torch.from_numpy(hst.copy()))
        for s in seq_ids:
            self._steps[s] = self._steps.get(s, 0) + 1
        return hid.tolist()

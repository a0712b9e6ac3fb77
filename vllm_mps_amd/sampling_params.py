"""Per-request sampling parameters -- same fields, defaults and validation as
the reference's ``SamplingParams`` (``core/sequence.py:23-61``)."""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass
class SamplingParams:
    """Controls how the next token is drawn from a logits row.

    temperature: 0 selects greedy argmax; otherwise logits are divided by it.
    top_k:       keep the k highest logits (0 disables the filter).
    top_p:       keep the smallest head of the sorted distribution whose mass
                 reaches top_p (1.0 disables the filter).
    max_tokens:  generation budget (used by the engine, not by the sampler).
    stop_sequences: stop strings (used by the engine, not by the sampler).
    """

    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    max_tokens: int = 128
    stop_sequences: list[str] = field(default_factory=list)

    def __post_init__(self) -> None:
        if self.temperature < 0.0:
            raise ValueError(f"SamplingParams: temperature must be >= 0.0, got {self.temperature}.")
        if self.top_k < 0:
            raise ValueError(f"SamplingParams: top_k must be >= 0, got {self.top_k}.")
        if not (0.0 < self.top_p <= 1.0):
            raise ValueError(f"SamplingParams: top_p must be in (0.0, 1.0], got {self.top_p}.")
        if self.max_tokens < 1:
            raise ValueError(f"SamplingParams: max_tokens must be >= 1, got {self.max_tokens}.")

"""MI355X-native decode-step token sampler (drop-in for vllm_mps's Sampler).

``Sampler`` and ``SamplingParams`` keep the reference's call surface
(``model/sampler.py``, ``core/sequence.py``); the arithmetic runs in
hand-written HIP kernels for gfx950 behind the C ABI in
``include/mis_sampler.h``.
"""
from .sampling_params import SamplingParams
from .sampler import Sampler, pack_params
from .engine_step import StepSampler

__all__ = ["Sampler", "SamplingParams", "StepSampler", "pack_params"]

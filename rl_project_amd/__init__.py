"""MI355X-native token-sampling path (drop-in for Forgeline's sampler).

Public API
----------
apply_sampling_filters, sample_from_logits, generate_tokens
    Reference-compatible functions (src/forgeline/models/generation/sampling.py).
sample_tokens, describe_rows, filtered_outputs, SamplerPlan
    Batched entry points with heterogeneous per-row parameters (SamplerPlan:
    prepared once, one launch per decode step, capturable in a graph).
BatchedSampler
    A decode group's sampling state on the device (inference/engine.py:114-139).
speculative_verify, SpecPlan, SpeculativeGenerator, MTPSpeculativeGenerator
    Speculative-decoding accept / resample and the generators over B sequences
    (models/generation/speculative.py).
lm_head_sample, LmHeadPlan
    lm_head and sampling in one call, without the [B, V] logits
    (models/transformer/model.py:190, :201).
token_logprobs_from_logits, entropy_from_logits, kl_full_distribution, row_stats
    Full-distribution log-prob / entropy / KL in one pass (models/policy.py,
    training/common/logprobs.py).
SamplingParams
    Per-request parameters with the reference's validation (inference/requests.py).
"""

from .params import GenerationSettings, SamplingParams, SamplingParamsError
from .sampling import (SampleOutput, SamplerPlan, SamplingError, apply_sampling_filters, describe_rows,
                       filtered_outputs, generate_tokens, sample_from_logits, sample_tokens)
from .speculative import MTPSpeculativeGenerator, SpeculativeGenerator, SpecOutput, SpecPlan, speculative_verify
from .engine import BatchedSampler
from .logprobs import RowStats, entropy_from_logits, kl_full_distribution, row_stats, token_logprobs_from_logits
from .lmhead import LmHeadOutput, LmHeadPlan, lm_head_sample

__all__ = [
    "apply_sampling_filters", "sample_from_logits", "generate_tokens",
    "sample_tokens", "describe_rows", "filtered_outputs", "SampleOutput", "SamplerPlan", "SamplingError",
    "speculative_verify", "SpeculativeGenerator", "MTPSpeculativeGenerator", "SpecOutput", "SpecPlan",
    "BatchedSampler", "row_stats", "RowStats", "token_logprobs_from_logits", "entropy_from_logits", "kl_full_distribution",
    "SamplingParams", "GenerationSettings", "SamplingParamsError",
    "lm_head_sample", "LmHeadPlan", "LmHeadOutput",
]

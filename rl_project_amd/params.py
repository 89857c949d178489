"""Sampling parameter carriers with the reference's defaults and validation.

``SamplingParams`` mirrors ``src/forgeline/inference/requests.py:23-41``
(defaults T=0.8, top_k=50, top_p/min_p off, penalty 1.0; the same four
checks).  ``GenerationSettings`` mirrors ``src/forgeline/core/protocols.py:18-31``.
``batch_tensors`` turns a list of per-request parameters into the per-row
device arrays the batched kernel reads (the inference engine's per-request
loop, ``inference/engine.py:114-139``, as one launch).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import torch


class SamplingParamsError(ValueError):
    """Invalid sampling parameters (the reference raises ServingError)."""


@dataclass
class SamplingParams:
    max_tokens: int = 64
    temperature: float = 0.8
    top_k: Optional[int] = 50
    top_p: Optional[float] = None
    min_p: Optional[float] = None
    repetition_penalty: float = 1.0
    stop_token_ids: List[int] = field(default_factory=list)

    def validate(self) -> None:
        """The checks of ``requests.py:33-41`` (min_p and the penalty are, as
        there, not validated)."""
        if self.max_tokens < 1:
            raise SamplingParamsError("max_tokens must be >= 1")
        if self.temperature < 0:
            raise SamplingParamsError("temperature must be >= 0")
        if self.top_p is not None and not 0 < self.top_p <= 1:
            raise SamplingParamsError("top_p must be in (0, 1]")
        if self.top_k is not None and self.top_k < 0:
            raise SamplingParamsError("top_k must be >= 0")


@dataclass
class GenerationSettings:
    max_new_tokens: int = 64
    temperature: float = 1.0
    top_k: Optional[int] = None
    top_p: Optional[float] = None
    stop_token_ids: Sequence[int] = ()


def batch_tensors(params: Sequence[SamplingParams], device: torch.device,
                  eos_token_id: Optional[int] = None) -> Dict[str, object]:
    """Per-row kernel arguments for a list of requests: off values are
    top_k 0, top_p 1.0, min_p 0.0, penalty 1.0; each row's stop set is its
    stop ids plus ``eos_token_id`` (``engine.py:123-125``)."""
    B = len(params)
    f32 = dict(dtype=torch.float32, device=device)
    stops = []
    for p in params:
        s = list(p.stop_token_ids)
        if eos_token_id is not None:
            s.append(int(eos_token_id))
        stops.append(s)
    return dict(
        temperature=torch.tensor([p.temperature for p in params], **f32),
        top_k=torch.tensor([p.top_k or 0 for p in params], dtype=torch.int32, device=device),
        top_p=torch.tensor([1.0 if p.top_p is None else p.top_p for p in params], **f32),
        min_p=torch.tensor([0.0 if p.min_p is None else p.min_p for p in params], **f32),
        repetition_penalty=torch.tensor([p.repetition_penalty for p in params], **f32),
        stop_ids=stops if any(stops) else None,
    ) if B else {}

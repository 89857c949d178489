"""Batched decode-group sampling with device-resident state: the replacement
for ``InferenceEngine._emit``'s per-request loop (reference
``inference/engine.py:114-139``, called per sequence from ``_decode_group``,
``:141-160``).

The reference samples each sequence of a decode group separately:
``apply_sampling_filters`` + ``sample_from_logits`` on a ``[1, V]`` slice and
``.item()`` per sequence, with the sequence's prompt + generated ids as the
penalty history (``engine.py:40,118-122``) and ``stop_token_ids`` plus the
EOS id as its stop set (``engine.py:123-125``).

``BatchedSampler`` keeps all of that on the device, per slot:

* the sampling parameters as arrays;
* the history ids, with capacity ``max_seq_len``;
* the stop set.

``step(logits)`` samples every active slot in one launch and appends the
tokens to the histories on the device. It returns device tensors; the caller
reads them back once per step, not once per sequence. Length limits,
cancellation and block allocation stay with the engine, as in the reference.
"""

from __future__ import annotations

from typing import Iterable, List, Optional, Sequence

import torch

from .params import SamplingParams
from .sampling import SampleOutput, sample_tokens


class BatchedSampler:
    """Device-resident sampling state of up to ``max_rows`` sequences.

    Slots ``0 .. n-1`` of a step are the first ``n`` rows of the logits, in
    the order the engine stacks its decode group; ``admit`` / ``release``
    manage which request holds which slot."""

    def __init__(self, max_rows: int, max_seq_len: int, vocab: int, device, *, eos_token_id: Optional[int] = None,
                 max_stop_ids: int = 8, generator: Optional[torch.Generator] = None):
        self.max_rows, self.max_seq_len, self.vocab = max_rows, max_seq_len, vocab
        self.device = torch.device(device)
        self.eos = eos_token_id
        self.generator = generator
        d = self.device
        self.temperature = torch.ones(max_rows, dtype=torch.float32, device=d)
        self.top_k = torch.zeros(max_rows, dtype=torch.int32, device=d)
        self.top_p = torch.ones(max_rows, dtype=torch.float32, device=d)
        self.min_p = torch.zeros(max_rows, dtype=torch.float32, device=d)
        self.rep_penalty = torch.ones(max_rows, dtype=torch.float32, device=d)
        self.history = torch.full((max_rows, max_seq_len), -1, dtype=torch.int32, device=d)
        self.hist_len = torch.zeros(max_rows, dtype=torch.int32, device=d)
        self.stop_ids = torch.full((max_rows, max_stop_ids + 1), -1, dtype=torch.int32, device=d)
        self.finished = torch.zeros(max_rows, dtype=torch.bool, device=d)
        self._host_len: List[int] = [0] * max_rows
        self._rows = torch.arange(max_rows, device=d)

    def admit(self, slot: int, params: SamplingParams, prompt_tokens: Sequence[int]) -> None:
        """Give ``slot`` to a new request: its parameters (validated as
        ``requests.py:33-41``), its prompt as the start of its history and its
        stop set (``stop_token_ids`` plus the EOS id)."""
        params.validate()
        n = len(prompt_tokens)
        if n >= self.max_seq_len:
            raise ValueError(f"prompt of {n} tokens does not fit max_seq_len {self.max_seq_len}")
        stops = sorted(set(int(s) for s in params.stop_token_ids) | ({self.eos} if self.eos is not None else set()))
        if len(stops) > self.stop_ids.size(1):
            raise ValueError(f"{len(stops)} stop ids exceed the {self.stop_ids.size(1)} slots per row")
        if any(t < 0 or t >= self.vocab for t in prompt_tokens):
            raise IndexError("prompt token outside the vocabulary")
        self.temperature[slot] = float(params.temperature)
        self.top_k[slot] = int(params.top_k or 0)
        self.top_p[slot] = float(params.top_p if params.top_p is not None else 1.0)
        self.min_p[slot] = float(params.min_p or 0.0)
        self.rep_penalty[slot] = float(params.repetition_penalty)
        row = torch.full((self.max_seq_len,), -1, dtype=torch.int32)
        row[:n] = torch.tensor(list(prompt_tokens), dtype=torch.int32)
        self.history[slot].copy_(row, non_blocking=False)
        self.hist_len[slot] = n
        srow = torch.full((self.stop_ids.size(1),), -1, dtype=torch.int32)
        if stops:
            srow[:len(stops)] = torch.tensor(stops, dtype=torch.int32)
        self.stop_ids[slot].copy_(srow)
        self.finished[slot] = False
        self._host_len[slot] = n

    def release(self, slot: int) -> None:
        self.finished[slot] = True

    def step(self, logits: torch.Tensor, uniforms: Optional[torch.Tensor] = None,
             return_logprobs: bool = False) -> SampleOutput:
        """Sample one token for each of the first ``logits.size(0)`` slots and
        append it to their histories (device only, no host synchronisation)."""
        n = logits.size(0)
        if n > self.max_rows:
            raise ValueError(f"{n} rows exceed max_rows {self.max_rows}")
        if max(self._host_len[:n], default=0) >= self.max_seq_len:
            raise ValueError("a history is full: retire the sequence before max_seq_len")
        if uniforms is None:
            uniforms = torch.rand(n, device=self.device, generator=self.generator)
        out = sample_tokens(logits, temperature=self.temperature[:n], top_k=self.top_k[:n], top_p=self.top_p[:n],
                            min_p=self.min_p[:n], repetition_penalty=self.rep_penalty[:n],
                            history=(self.history[:n], self.hist_len[:n]), stop_ids=self.stop_ids[:n],
                            uniforms=uniforms, finished=self.finished[:n], return_logprobs=return_logprobs)
        # append to the histories on the device
        rows = self._rows[:n]
        self.history[rows, self.hist_len[:n].long()] = out.tokens.to(torch.int32)
        self.hist_len[:n] += 1
        self.finished[:n] = out.finished
        for i in range(n):
            self._host_len[i] += 1
        return out

    def history_of(self, slot: int) -> List[int]:
        """Prompt + generated ids of a slot (reads the device: for tests and retirement)."""
        return self.history[slot, : int(self.hist_len[slot])].tolist()

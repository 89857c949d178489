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

``step(logits)`` samples every row in one launch; the kernel also sets the
finished flags and appends the tokens to the histories (no host
synchronisation, no other kernel). It returns device tensors; the caller
reads them back once per step, not once per sequence. Length limits,
cancellation and block allocation stay with the engine, as in the reference.
"""

from __future__ import annotations

from typing import Dict, Iterable, List, Optional, Sequence, Tuple

import torch

from .params import SamplingParams
from . import _lib
from .sampling import SampleOutput, _Call, _check_logits


class BatchedSampler:
    """Device-resident sampling state of up to ``max_rows`` sequences.

    Row ``i`` of a step's logits belongs to slot ``i`` (or to ``slots[i]`` when
    the step names its slots); ``admit`` / ``release`` manage which request
    holds which slot.  A step is one ``fl_sample`` launch: the kernel samples
    every row, sets the finished flags in place and appends each token to its
    slot's history (``FL_FLAG_APPEND_HISTORY``); nothing is synchronised with
    the host and nothing is allocated (the argument block and the output
    buffers are kept per row count and reused, so a step's outputs are valid
    until the next step)."""

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
        # uint8, updated in place by the kernel (finished_in and out_finished)
        self.finished_u8 = torch.ones(max_rows, dtype=torch.uint8, device=d)
        self._plans: Dict[Tuple[int, torch.dtype, int, int, bool], _Call] = {}

    @property
    def finished(self) -> torch.Tensor:
        """bool [max_rows]: slots that produced a stop id or were released."""
        return self.finished_u8.view(torch.bool)

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
        self.finished_u8[slot] = 0

    def release(self, slot: int) -> None:
        """Retire ``slot``: it is finished (a row of a later step that still
        maps to it samples but appends nothing) and its history is emptied."""
        self.finished_u8[slot] = 1
        self.hist_len[slot] = 0

    def _plan(self, n: int, logits: torch.Tensor, want_logprob: bool) -> _Call:
        key = (n, logits.dtype, logits.size(1), logits.stride(0), want_logprob)
        call = self._plans.get(key)
        if call is None:
            call = _Call(logits, temperature=self.temperature[:n], top_k=self.top_k[:n], top_p=self.top_p[:n],
                         min_p=self.min_p[:n], repetition_penalty=self.rep_penalty[:n],
                         history=(self.history[:n], self.hist_len[:n]), stop_ids=self.stop_ids[:n],
                         uniforms=torch.zeros(n, dtype=torch.float32, device=self.device),
                         finished=self.finished_u8[:n], out_finished=self.finished_u8[:n],
                         flags=_lib.FL_FLAG_APPEND_HISTORY, want_logprob=want_logprob)
            # the state tensors are used in place, never copied
            assert call.hist.data_ptr() == self.history.data_ptr() and call.fin_in.data_ptr() == \
                self.finished_u8.data_ptr()
            self._plans[key] = call
        return call

    def step(self, logits: torch.Tensor, uniforms: Optional[torch.Tensor] = None, return_logprobs: bool = False,
             slots: Optional[torch.Tensor] = None) -> SampleOutput:
        """Sample one token for each row of ``logits`` (row i: slot i, or
        ``slots[i]``), mark the rows that produced a stop id as finished and
        append the tokens of unfinished rows to their histories, in one launch
        with no host synchronisation.  ``status`` of the output carries the
        per-row FL_ROW_* bits for the caller to read with the tokens."""
        n = logits.size(0)
        if n > self.max_rows:
            raise ValueError(f"{n} rows exceed max_rows {self.max_rows}")
        if uniforms is None:
            uniforms = torch.rand(n, device=self.device, generator=self.generator)
        if slots is not None:
            return self._step_slots(logits, uniforms, return_logprobs, slots)
        logits = _check_logits(logits)
        call = self._plan(n, logits, return_logprobs)
        if uniforms.dtype != torch.float32 or not uniforms.is_contiguous() or uniforms.numel() != n:
            raise ValueError("uniforms must be a contiguous float32 tensor with one draw per row")
        call.args.logits = logits.data_ptr()
        call.args.uniforms = uniforms.data_ptr()
        call.keep = (logits, uniforms)   # alive until the kernel has read them
        call.run()
        # 16-bit rows where one value fills more than 65535 positions: the
        # exact-count repeat (a kernel that leaves every other row alone)
        if logits.size(1) > 0xFFFF:
            call.run_exact_for_limited()
        return SampleOutput(call.tokens, call.finished[:n].view(torch.bool), call.status, call.logprob)

    def _step_slots(self, logits, uniforms, return_logprobs, slots) -> SampleOutput:
        """A decode group whose rows map to arbitrary slots: gather the slots'
        state, sample with the append, scatter the state back (a few small
        device copies; no host synchronisation)."""
        idx = slots.to(device=self.device, dtype=torch.long)
        hist = self.history.index_select(0, idx)
        hlen = self.hist_len.index_select(0, idx)
        fin = self.finished_u8.index_select(0, idx)
        call = _Call(logits, temperature=self.temperature[idx], top_k=self.top_k[idx], top_p=self.top_p[idx],
                     min_p=self.min_p[idx], repetition_penalty=self.rep_penalty[idx], history=(hist, hlen),
                     stop_ids=self.stop_ids[idx], uniforms=uniforms, finished=fin, out_finished=fin,
                     flags=_lib.FL_FLAG_APPEND_HISTORY, want_logprob=return_logprobs).run()
        if logits.size(1) > 0xFFFF:
            call.run_exact_for_limited()
        self.history.index_copy_(0, idx, hist)
        self.hist_len.index_copy_(0, idx, hlen)
        self.finished_u8.index_copy_(0, idx, fin)
        return SampleOutput(call.tokens, fin.view(torch.bool), call.status, call.logprob)

    def history_of(self, slot: int) -> List[int]:
        """Prompt + generated ids of a slot (reads the device: for tests and retirement)."""
        return self.history[slot, : int(self.hist_len[slot])].tolist()

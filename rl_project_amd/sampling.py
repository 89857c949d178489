"""MI355X drop-in for the reference's token sampler.

Mirrors ``src/forgeline/models/generation/sampling.py`` (same function names,
arguments and return shapes) and adds the batched entry point
``sample_tokens`` with heterogeneous per-row parameters, per-row histories and
stop sets (the per-request loop of ``src/forgeline/inference/engine.py:114-139``
in one launch).  Every call runs the hand-written gfx950 kernels of
``libflsampler.so`` through its C ABI; device tensors only, no CPU fallback.

Selection convention (replaces ``torch.multinomial``, ``sampling.py:61``):
inverse CDF over the filtered softmax, visiting tokens by descending filtered
value with ties by ascending vocabulary index, driven by one caller-supplied
uniform per row (drawn from torch's generator when not supplied).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Iterable, List, Optional, Sequence, Tuple, Union

import torch
import torch.nn.functional as F  # noqa: F401  (kept for API parity with the reference module)

from . import _lib
from ._lib import FL_FLAG_NO_SELECT, ROW_DESC_BYTES, SampleArgs, check, lib, ptr

_DTYPES = {torch.float32: _lib.FL_DTYPE_F32, torch.bfloat16: _lib.FL_DTYPE_BF16, torch.float16: _lib.FL_DTYPE_F16}

PerRow = Union[None, float, int, Sequence, torch.Tensor]


class SamplingError(RuntimeError):
    """A row could not be sampled (NaN logits, bad history id, everything filtered)."""


@dataclass
class SampleOutput:
    tokens: torch.Tensor          # int64 [B]; -1 for rows with a non-zero status
    finished: torch.Tensor        # bool [B]
    status: torch.Tensor          # int32 [B]; FL_ROW_* bits
    logprobs: Optional[torch.Tensor] = None   # float32 [B]
    desc: Optional[torch.Tensor] = None       # uint8 [B, 32]: fl_row_desc records


def _check_logits(logits: torch.Tensor) -> torch.Tensor:
    if not isinstance(logits, torch.Tensor):
        raise TypeError("logits must be a torch.Tensor")
    if logits.device.type != "cuda":
        raise ValueError("the MI355X sampler needs logits on a ROCm device (no CPU fallback)")
    if logits.dim() != 2:
        raise ValueError(f"logits must be [B, V], got {tuple(logits.shape)}")
    if logits.dtype not in _DTYPES:
        raise NotImplementedError(f"logits dtype {logits.dtype} is not supported (float32, bfloat16, float16)")
    if logits.stride(-1) != 1 or (logits.size(0) > 1 and logits.stride(0) < logits.size(1)):
        logits = logits.contiguous()
    return logits


def _per_row(value: PerRow, B: int, dtype: torch.dtype, device: torch.device, off) -> torch.Tensor:
    if value is None:
        value = off
    if isinstance(value, torch.Tensor):
        t = value.to(device=device, dtype=dtype).reshape(-1)
        if t.numel() == 1:
            t = t.expand(B)
    elif isinstance(value, (int, float)):
        return torch.full((B,), value, dtype=dtype, device=device)
    else:
        t = torch.tensor([off if v is None else v for v in value], dtype=dtype, device=device)
    if t.numel() != B:
        raise ValueError(f"per-row parameter has {t.numel()} entries for {B} rows")
    return t.contiguous()


def _history_tensor(history, B: int, V: int, device: torch.device) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor], int]:
    """Pack per-row histories into ([B, H] int32, [B] int32 lengths, row stride)."""
    if history is None:
        return None, None, 0
    if (isinstance(history, tuple) and len(history) == 2 and isinstance(history[0], torch.Tensor)
            and isinstance(history[1], torch.Tensor)):
        # device-resident (ids [B, H] int32, lengths [B] int32): used as they are
        h, lens = history
        if h.dim() != 2 or h.size(0) != B or lens.numel() != B or h.dtype != torch.int32 or lens.dtype != torch.int32:
            raise ValueError("history (ids, lengths) must be int32 [B, H] and int32 [B]")
        if h.size(1) > _lib.FL_MAX_HISTORY:
            raise NotImplementedError(f"history of {h.size(1)} ids exceeds {_lib.FL_MAX_HISTORY}")
        if h.stride(1) != 1:
            h = h.contiguous()
        return h, lens.contiguous(), h.stride(0) if B > 1 else h.size(1)
    if isinstance(history, torch.Tensor):
        h = history.to(device=device, dtype=torch.int32)
        if h.dim() == 1:
            h = h.unsqueeze(0).expand(B, -1)
        h = h.contiguous()
        lens = torch.full((B,), h.size(1), dtype=torch.int32, device=device)
        return h, lens, h.size(1)
    rows: List[List[int]] = [list(r) if r is not None else [] for r in history]
    if len(rows) != B:
        raise ValueError(f"history has {len(rows)} rows for {B} logits rows")
    H = max([len(r) for r in rows] + [1])
    if H > _lib.FL_MAX_HISTORY:
        raise NotImplementedError(f"history of {H} ids exceeds {_lib.FL_MAX_HISTORY}")
    buf = torch.full((B, H), -1, dtype=torch.int32)
    for b, r in enumerate(rows):
        if r:
            buf[b, :len(r)] = torch.tensor(r, dtype=torch.int32)
    lens = torch.tensor([len(r) for r in rows], dtype=torch.int32)
    return buf.to(device), lens.to(device), H


def _stop_tensor(stop_ids, B: int, device: torch.device) -> Tuple[Optional[torch.Tensor], int, int]:
    if stop_ids is None:
        return None, 0, 0
    if isinstance(stop_ids, torch.Tensor):
        s = stop_ids.to(device=device, dtype=torch.int32)
        if s.dim() == 1:
            return s.contiguous(), 0, s.numel()
        return s.contiguous(), s.size(1), s.size(1)
    seq = list(stop_ids)
    if seq and isinstance(seq[0], (list, tuple, set)):
        S = max([len(r) for r in seq] + [1])
        buf = torch.full((B, S), -1, dtype=torch.int32)
        for b, r in enumerate(seq):
            r = list(r)
            if r:
                buf[b, :len(r)] = torch.tensor(r, dtype=torch.int32)
        return buf.to(device), S, S
    if not seq:
        return None, 0, 0
    return torch.tensor(seq, dtype=torch.int32, device=device), 0, len(seq)


class _Call:
    """Argument block of one fl_sample call with the tensors it points to."""

    def __init__(self, logits: torch.Tensor, *, temperature: PerRow = 1.0, top_k: PerRow = None,
                 top_p: PerRow = None, min_p: PerRow = None, repetition_penalty: PerRow = 1.0, history=None,
                 stop_ids=None, uniforms: Optional[torch.Tensor] = None, finished: Optional[torch.Tensor] = None,
                 softcap: float = 0.0, flags: int = 0, want_logprob: bool = False, want_desc: bool = False,
                 uniform_div: int = 1, out_finished: Optional[torch.Tensor] = None):
        self.logits = logits = _check_logits(logits)
        B, V = logits.shape
        dev = logits.device
        self.B, self.V = B, V
        self.T = _per_row(temperature, B, torch.float32, dev, 1.0)
        self.K = _per_row(top_k, B, torch.int32, dev, 0)
        self.P = _per_row(top_p, B, torch.float32, dev, 1.0)
        self.MP = _per_row(min_p, B, torch.float32, dev, 0.0)
        self.RP = _per_row(repetition_penalty, B, torch.float32, dev, 1.0)
        self.hist, self.hist_len, self.hist_ld = _history_tensor(history, B, V, dev)
        self.stop, self.stop_ld, self.n_stop = _stop_tensor(stop_ids, B, dev)
        select = not (flags & FL_FLAG_NO_SELECT)
        uniform_div = max(1, int(uniform_div))
        n_draws = (B + uniform_div - 1) // uniform_div
        if uniforms is None and select:
            uniforms = torch.rand(n_draws, device=dev, dtype=torch.float32)
        self.U = None if uniforms is None else uniforms.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
        if self.U is not None and self.U.numel() != n_draws:
            raise ValueError(f"uniforms has {self.U.numel()} entries for {B} rows ({n_draws} draws)")
        if flags & _lib.FL_FLAG_APPEND_HISTORY and (self.hist is None or self.hist_ld <= 0 or B > 1 and
                                                    self.hist.stride(0) != self.hist_ld):
            raise ValueError("appending to the histories needs a per-row (ids, lengths) history")
        self.fin_in = None if finished is None else finished.to(device=dev, dtype=torch.uint8).reshape(-1).contiguous()
        self.tokens = torch.empty(B, dtype=torch.int64, device=dev)
        # (out_finished may be the finished_in buffer itself: each row reads its
        # flag before writing it)
        self.finished = out_finished if out_finished is not None else torch.empty(B, dtype=torch.uint8, device=dev)
        self.status = torch.empty(B, dtype=torch.int32, device=dev)
        self.logprob = torch.empty(B, dtype=torch.float32, device=dev) if want_logprob else None
        self.desc = torch.empty(B, ROW_DESC_BYTES, dtype=torch.uint8, device=dev) if want_desc else None
        a = SampleArgs()
        a.struct_size = ctypes.sizeof(SampleArgs)
        a.dtype = _DTYPES[logits.dtype]
        a.logits = logits.data_ptr()
        a.batch, a.vocab, a.ld = B, V, logits.stride(0) if B > 1 else V
        a.temperature, a.top_k, a.top_p, a.min_p, a.rep_penalty = (
            ptr(self.T), ptr(self.K), ptr(self.P), ptr(self.MP), ptr(self.RP))
        a.softcap = float(softcap or 0.0)
        a.flags = flags
        a.hist_ids, a.hist_ld, a.hist_len = ptr(self.hist), self.hist_ld, ptr(self.hist_len)
        a.stop_ids, a.stop_ld, a.n_stop = ptr(self.stop), self.stop_ld, self.n_stop
        a.uniforms, a.finished_in = ptr(self.U), ptr(self.fin_in)
        a.out_token, a.out_finished, a.out_status = ptr(self.tokens), ptr(self.finished), ptr(self.status)
        a.out_logprob, a.out_desc = ptr(self.logprob), ptr(self.desc)
        a.uniform_div = uniform_div
        self.args = a
        self.device = dev

    @property
    def stream(self) -> int:
        """The device's current stream (read at each launch, as torch ops do:
        a launch under graph capture is recorded into the graph)."""
        return _lib.stream_handle(self.device)

    def run(self) -> "_Call":
        check(lib().fl_sample(ctypes.byref(self.args), self.stream), "fl_sample")
        return self

    def run_exact_for_limited(self) -> "_Call":
        """Repeat the call for the rows it left at FL_ROW_LIMIT with the
        exact-count kernel (16-bit rows where one value fills more than 65535
        positions); every other row keeps its outputs.  Stream-ordered, no
        host synchronisation (the kernel reads the status)."""
        if self.logits.dtype == torch.float32:
            return self
        flags = self.args.flags
        self.args.flags = flags | _lib.FL_FLAG_EXACT_COUNTS | _lib.FL_FLAG_ONLY_LIMITED
        try:
            check(lib().fl_sample(ctypes.byref(self.args), self.stream), "fl_sample")
        finally:
            self.args.flags = flags
        return self

    def run_checked(self) -> "_Call":
        """run(), then the exact-count repeat if a 16-bit row reports
        FL_ROW_LIMIT (synchronises with the host to read the status)."""
        self.run()
        if self.logits.dtype != torch.float32 and bool(((self.status & _lib.FL_ROW_LIMIT) != 0).any()):
            self.run_exact_for_limited()
        return self


class SamplerPlan:
    """A prepared ``sample_tokens`` call: arguments and output buffers are
    built once, each ``launch()`` only enqueues the kernel (no allocation, no
    host synchronisation) -- for decode loops that resample the same buffers.
    Reads ``logits`` and the parameter tensors at launch time, so callers may
    overwrite them in place between launches.  Each launch goes to the
    device's current stream, so a launch inside ``torch.cuda.graph`` capture
    is recorded into the graph (the kernels allocate, copy and clear
    nothing)."""

    def __init__(self, logits: torch.Tensor, exact_repeat: bool = True, **kw):
        want_logprob = kw.pop("return_logprobs", False)
        want_desc = kw.pop("return_desc", False)
        self._call = _Call(logits, flags=0, want_logprob=want_logprob, want_desc=want_desc,
                           finished=kw.pop("finished", None), uniforms=kw.pop("uniforms", None), **kw)
        self._fn = lib().fl_sample
        self._argp = ctypes.byref(self._call.args)
        # exact_repeat (default): every launch also enqueues the exact-count
        # repeat for rows left at FL_ROW_LIMIT (one more kernel; no host
        # synchronisation).  Only 16-bit rows longer than 65535 values can
        # hold more equal values than a 16-bit counter; a caller that checks
        # the status itself may turn it off.
        self._exact = exact_repeat and logits.dtype != torch.float32 and logits.size(-1) > 0xFFFF

    def launch(self) -> None:
        rc = self._fn(self._argp, self._call.stream)
        if rc:
            check(rc, "fl_sample")
        if self._exact:
            self._call.run_exact_for_limited()

    @property
    def output(self) -> SampleOutput:
        c = self._call
        return SampleOutput(c.tokens, c.finished.bool(), c.status, c.logprob, c.desc)


def _raise_on_status(status: torch.Tensor, allowed: int = 0) -> None:
    bad = status & ~allowed
    if bool((bad != 0).any()):
        rows = torch.nonzero(bad).flatten().tolist()
        codes = 0
        for v in bad[bad != 0].tolist():
            codes |= int(v)
        names = [n for bit, n in _lib.ROW_STATUS_NAMES.items() if codes & bit]
        raise SamplingError(f"rows {rows[:8]}{'...' if len(rows) > 8 else ''} failed: {', '.join(names) or codes}")


# ---------------------------------------------------------------------------
# Batched entry point
# ---------------------------------------------------------------------------

def sample_tokens(
    logits: torch.Tensor,
    *,
    temperature: PerRow = 1.0,
    top_k: PerRow = None,
    top_p: PerRow = None,
    min_p: PerRow = None,
    repetition_penalty: PerRow = 1.0,
    history=None,
    stop_ids=None,
    uniforms: Optional[torch.Tensor] = None,
    finished: Optional[torch.Tensor] = None,
    softcap: float = 0.0,
    return_logprobs: bool = False,
    return_desc: bool = False,
    check_status: bool = True,
) -> SampleOutput:
    """Filter and sample one token per row of ``logits`` [B, V] in one launch.

    Per-row parameters accept a scalar, a sequence (None entries mean "off") or
    a device tensor.  ``history``: per-row token-id lists (or a [B, H] / [H]
    tensor, or a device-resident pair (ids int32 [B, H], lengths int32 [B]))
    for the repetition penalty; ``stop_ids``: one shared list, per-row
    lists, or a [S] / [B, S] tensor; ``uniforms``: float32 [B] in [0, 1).
    Equivalent to ``engine.py:118-127`` applied to every row: the filtered
    logits of ``apply_sampling_filters``, ``sample_from_logits``, the stop test
    and (``return_logprobs``) the post-filter log-probability of the token."""
    call = _Call(logits, temperature=temperature, top_k=top_k, top_p=top_p, min_p=min_p,
                 repetition_penalty=repetition_penalty, history=history, stop_ids=stop_ids, uniforms=uniforms,
                 finished=finished, softcap=softcap, flags=0, want_logprob=return_logprobs,
                 want_desc=return_desc)
    if check_status:
        call.run_checked()
        _raise_on_status(call.status)
    else:
        call.run()
    return SampleOutput(call.tokens, call.finished.bool(), call.status, call.logprob, call.desc)


def describe_rows(logits: torch.Tensor, **kw) -> Tuple[torch.Tensor, torch.Tensor]:
    """Descriptors of the filtered distribution of every row (no selection)."""
    call = _Call(logits, flags=FL_FLAG_NO_SELECT, want_logprob=False, want_desc=True, uniforms=None,
                 finished=None, **kw).run_checked()
    return call.desc, call.status


def filtered_outputs(logits: torch.Tensor, *, want_filtered: bool = True, want_probs: bool = False,
                     want_mask: bool = False, **kw):
    """(filtered logits, probabilities, keep bit-mask, status) of every row; any may be skipped."""
    call = _Call(logits, flags=FL_FLAG_NO_SELECT, want_logprob=False, want_desc=True, uniforms=None,
                 finished=None, **kw).run_checked()
    B, V = call.B, call.V
    dev = call.logits.device
    out = torch.empty(B, V, dtype=call.logits.dtype, device=dev) if want_filtered else None
    probs = torch.empty(B, V, dtype=torch.float32, device=dev) if want_probs else None
    mask = torch.empty(B, (V + 31) // 32, dtype=torch.int32, device=dev) if want_mask else None
    check(lib().fl_apply_filter(ctypes.byref(call.args), ptr(call.desc), ptr(out), V, ptr(probs), ptr(mask),
                                call.stream), "fl_apply_filter")
    return out, probs, mask, call.status


# ---------------------------------------------------------------------------
# Reference-compatible functions (sampling.py:16-132)
# ---------------------------------------------------------------------------

def _normalise_past(past_tokens: Optional[Sequence[int]], V: int) -> Optional[List[int]]:
    """``torch.tensor(list(past)).unique()`` indexing semantics: negative ids
    wrap once, anything else outside [0, V) is an IndexError."""
    if not past_tokens:
        return None
    ids = []
    for t in past_tokens:
        t = int(t)
        if t < 0:
            t += V
        if t < 0 or t >= V:
            raise IndexError(f"history id {t} is out of bounds for vocabulary {V}")
        ids.append(t)
    return ids


def apply_sampling_filters(
    logits: torch.Tensor,
    temperature: float = 1.0,
    top_k: Optional[int] = None,
    top_p: Optional[float] = None,
    min_p: Optional[float] = None,
    repetition_penalty: float = 1.0,
    past_tokens: Optional[Sequence[int]] = None,
) -> torch.Tensor:
    """Return filtered logits ``[B, V]`` (reference ``sampling.py:16-53``).

    Same arguments and result as the reference: a new tensor in the input
    dtype with removed entries at ``-inf``; ``past_tokens`` is one id list
    shared by every row.  ``temperature <= 0`` leaves logits unscaled."""
    logits = _check_logits(logits)
    B, V = logits.shape
    past = _normalise_past(past_tokens, V) if repetition_penalty != 1.0 else None
    history = torch.tensor(past, dtype=torch.int32, device=logits.device) if past else None
    out, _, _, status = filtered_outputs(
        logits, temperature=temperature, top_k=top_k if (top_k is not None and top_k > 0) else 0,
        top_p=top_p if top_p is not None else 1.0, min_p=min_p if min_p is not None else 0.0,
        repetition_penalty=repetition_penalty, history=history, stop_ids=None, softcap=0.0)
    # an all-filtered row is returned as all -inf, as the reference returns it
    _raise_on_status(status, allowed=_lib.FL_ROW_ALL_MASKED)
    return out


def sample_from_logits(logits: torch.Tensor, temperature: float = 1.0,
                       uniforms: Optional[torch.Tensor] = None,
                       generator: Optional[torch.Generator] = None) -> torch.Tensor:
    """Greedy when ``temperature <= 0`` else one draw from ``softmax(logits)``;
    returns ``[B, 1]`` int64 (reference ``sampling.py:56-61``).  ``uniforms``
    (float32 [B]) drive the inverse-CDF draw; drawn from ``generator`` if None."""
    logits = _check_logits(logits)
    B = logits.size(0)
    if uniforms is None and temperature > 0:
        uniforms = torch.rand(B, device=logits.device, generator=generator)
    out = sample_tokens(logits, temperature=1.0 if temperature > 0 else 0.0, uniforms=uniforms)
    return out.tokens.view(B, 1)


@torch.no_grad()
def generate_tokens(
    model,
    idx: torch.Tensor,
    max_new_tokens: int,
    temperature: float = 1.0,
    top_k: Optional[int] = None,
    top_p: Optional[float] = None,
    min_p: Optional[float] = None,
    repetition_penalty: float = 1.0,
    use_cache: bool = True,
    stop_token_ids: Iterable[int] = (),
    return_logprobs: bool = False,
    generator: Optional[torch.Generator] = None,
):
    """Autoregressive sampling for a batch of prompts ``[B, T]`` (reference
    ``sampling.py:64-132``): same model protocol (``prefill``/``step`` or a
    full forward), same stopping rule (the whole batch stops once every row
    produced a stop id) and the same penalty scope (the reference penalises
    only when ``B == 1``, with the prompt plus generated ids as history).
    Filtering, selection, the stop test and the log-probability are one fused
    launch per step."""
    stop = sorted(set(int(t) for t in stop_token_ids))
    B = idx.size(0)
    dev = idx.device
    pen_on = repetition_penalty != 1.0 and B == 1
    past: Optional[List[int]] = idx[0].tolist() if pen_on else None
    generated: List[torch.Tensor] = []
    logprobs: List[torch.Tensor] = []
    finished = torch.zeros(B, dtype=torch.bool, device=dev)
    block_size = model.spec.block_size
    stop_t = torch.tensor(stop, dtype=torch.int32, device=dev) if stop else None
    kw = dict(temperature=temperature, top_k=top_k if (top_k is not None and top_k > 0) else 0,
              top_p=top_p if top_p is not None else 1.0, min_p=min_p if min_p is not None else 0.0,
              repetition_penalty=repetition_penalty if pen_on else 1.0)

    def _sample(logits: torch.Tensor) -> torch.Tensor:
        nonlocal finished
        hist = [past] if pen_on else None
        u = torch.rand(B, device=dev, generator=generator) if temperature > 0 else None
        out = sample_tokens(logits, history=hist, stop_ids=stop_t, uniforms=u, finished=finished,
                            return_logprobs=return_logprobs, **kw)
        finished = out.finished
        if return_logprobs:
            logprobs.append(out.logprobs)
        return out.tokens.view(B, 1)

    if use_cache and idx.size(1) < block_size:
        logits, cache = model.prefill(idx)
        position = idx.size(1)
        for _ in range(max_new_tokens):
            nxt = _sample(logits)
            generated.append(nxt)
            if past is not None:
                past.append(int(nxt.item()))
            if bool(finished.all()) or position >= block_size:
                break
            logits, cache = model.step(nxt, cache, position)
            position += 1
    else:
        seq = idx
        for _ in range(max_new_tokens):
            ctx = seq if seq.size(1) <= block_size else seq[:, -block_size:]
            logits, _ = model(ctx)
            nxt = _sample(logits[:, -1, :])
            generated.append(nxt)
            seq = torch.cat([seq, nxt], dim=1)
            if past is not None:
                past.append(int(nxt.item()))
            if bool(finished.all()):
                break

    out = torch.cat([idx] + generated, dim=1) if generated else idx
    if return_logprobs:
        lp = torch.stack(logprobs, dim=1) if logprobs else torch.zeros(B, 0, device=dev)
        return out, lp
    return out

"""lm_head with the sampler fused into its epilogue (``fl_lm_head_sample``).

The decode step of the reference computes ``logits = lm_head(h[:, -1, :])``
(``transformer/model.py:190``, ``:201``) and samples them
(``generation/sampling.py:16-61``).  For rows that use top-k (1 to 64),
``LmHeadPlan`` does both without ever writing the ``[B, V]`` logits: the
MFMA GEMM's epilogue applies soft-cap, penalty and temperature and keeps only
the values that can be among each row's k largest; a second kernel samples
each row from those with ``fl_sample``'s rules.

Rows the fused kernels cannot decide (top-k off or above 64, more than 4096
values tied above the threshold) report ``FL_ROW_LIMIT``; ``lm_head_sample``
then samples them with ``fl_sample`` over the logits the GEMM computed (the
same GEMM run with its logits output on).

On MI355X the fused step is slower than ``torch.nn.functional.linear``
(hipBLASLt) followed by ``fl_sample`` at every batch size measured (B = 1 to
64 at D = 4096, V = 128256: 230-268 us against 220-243 us).  So
``lm_head_sample`` takes the unfused path unless asked for the fused one
(``fused=True``), which callers that cannot hold the ``[B, V]`` logits use.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import LmHeadArgs, check, lib, ptr
from .sampling import PerRow, _history_tensor, _per_row, _raise_on_status, sample_tokens


def fused_is_faster(batch: int, dim: int, vocab: int) -> bool:
    """Whether the fused kernels beat ``linear`` + ``fl_sample`` for this shape:
    the crossover measured on MI355X.  At D = 4096, V = 128256 and every B from
    1 to 64 the unfused path was faster (by 10 us at B = 1, 25 us at B = 64),
    so no measured shape picks the fused path."""
    return False


@dataclass
class LmHeadOutput:
    tokens: torch.Tensor                 # int64 [B]
    status: torch.Tensor                 # int32 [B] (FL_ROW_* bits of the fused path)
    logprobs: Optional[torch.Tensor]     # float32 [B] or None
    logits: Optional[torch.Tensor]       # bf16 [B, V] when requested


class LmHeadPlan:
    """A prepared fused lm_head + sampling step for ``hidden`` [B, D] bf16 and
    ``weight`` [V, D] bf16 (the lm_head weight; tied to the token embedding
    in the reference model).  Buffers and the argument block are built once;
    ``launch()`` enqueues the kernels (four, five with a penalty) on the
    device's current stream with no allocation and no host synchronisation,
    reading ``hidden``, the parameters and the uniforms at launch time (a
    decode loop may overwrite them in place, or capture ``launch()`` in a
    graph)."""

    def __init__(self, hidden: torch.Tensor, weight: torch.Tensor, *, temperature: PerRow = 1.0,
                 top_k: PerRow = 50, top_p: PerRow = None, min_p: PerRow = None,
                 repetition_penalty: PerRow = None, history=None, softcap: float = 0.0,
                 uniforms: Optional[torch.Tensor] = None, generator: Optional[torch.Generator] = None,
                 return_logprobs: bool = False, return_logits: bool = False):
        if hidden.dim() != 2 or weight.dim() != 2 or hidden.size(1) != weight.size(1):
            raise ValueError(f"hidden [B, D] and weight [V, D] expected, got {tuple(hidden.shape)} and "
                             f"{tuple(weight.shape)}")
        if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
            raise NotImplementedError("the fused lm_head path takes bf16 hidden states and weights")
        if not hidden.is_cuda or hidden.device != weight.device:
            raise ValueError("hidden and weight must be on the same GPU")
        # (the kernels address the hidden states with 32-bit offsets: a
        # strided view whose rows span more than 2^29 elements, such as the
        # last position of [B, T, D] prefill states, is copied first)
        if hidden.stride(1) != 1 or (hidden.size(0) > 1 and hidden.size(0) * hidden.stride(0) > (1 << 29)):
            hidden = hidden.contiguous()
        if not weight.is_contiguous():
            raise ValueError("weight must be contiguous")
        B, D = hidden.shape
        V = weight.size(0)
        dev = hidden.device
        self.B, self.D, self.V = B, D, V
        self.hidden, self.weight = hidden, weight
        self.T = _per_row(temperature, B, torch.float32, dev, 1.0)
        self.K = _per_row(top_k, B, torch.int32, dev, 0)
        self.P = _per_row(top_p, B, torch.float32, dev, 1.0)
        self.MP = _per_row(min_p, B, torch.float32, dev, 0.0)
        self.RP = _per_row(repetition_penalty, B, torch.float32, dev, 1.0)
        self.hist, self.hist_len, self.hist_ld = _history_tensor(history, B, V, dev)
        if uniforms is None:
            uniforms = torch.rand(B, device=dev, generator=generator)
        self.U = uniforms.to(device=dev, dtype=torch.float32).contiguous()
        self.tokens = torch.empty(B, dtype=torch.int64, device=dev)
        self.status = torch.empty(B, dtype=torch.int32, device=dev)
        self.logprob = torch.empty(B, dtype=torch.float32, device=dev) if return_logprobs else None
        self.logits = torch.empty(B, V, dtype=torch.bfloat16, device=dev) if return_logits else None
        n = ctypes.c_size_t(0)
        check(lib().fl_lm_head_workspace_bytes(B, V, ctypes.byref(n)), "fl_lm_head_workspace_bytes")
        self._ws = torch.empty(max(int(n.value), 256), dtype=torch.uint8, device=dev)
        a = LmHeadArgs()
        a.struct_size = ctypes.sizeof(LmHeadArgs)
        a.dtype = _lib.FL_DTYPE_BF16
        a.hidden, a.weight = hidden.data_ptr(), weight.data_ptr()
        a.batch, a.dim, a.vocab, a.ld_hidden = B, D, V, hidden.stride(0) if B > 1 else D
        a.temperature, a.top_k, a.top_p, a.min_p = ptr(self.T), ptr(self.K), ptr(self.P), ptr(self.MP)
        a.repetition_penalty = ptr(self.RP) if self.hist is not None else None
        a.hist_ids, a.hist_len, a.hist_ld = ptr(self.hist), ptr(self.hist_len), self.hist_ld
        a.softcap = float(softcap or 0.0)
        a.uniforms = ptr(self.U)
        a.out_token, a.out_status, a.out_logprob, a.out_logits = (ptr(self.tokens), ptr(self.status),
                                                                 ptr(self.logprob), ptr(self.logits))
        a.workspace, a.workspace_bytes = self._ws.data_ptr(), self._ws.numel()
        self.args = a
        self._argp = ctypes.byref(a)
        self._fn = lib().fl_lm_head_sample
        self._dev = dev
        self.softcap = a.softcap
        self.history = history

    def launch(self) -> None:
        rc = self._fn(self._argp, _lib.stream_handle(self._dev))   # the current stream (graph capture records it)
        if rc:
            check(rc, "fl_lm_head_sample")

    @property
    def output(self) -> LmHeadOutput:
        return LmHeadOutput(self.tokens, self.status, self.logprob, self.logits)


def lm_head_sample(hidden: torch.Tensor, weight: torch.Tensor, *, temperature: PerRow = 1.0, top_k: PerRow = 50,
                   top_p: PerRow = None, min_p: PerRow = None, repetition_penalty: PerRow = None, history=None,
                   softcap: float = 0.0, uniforms: Optional[torch.Tensor] = None,
                   generator: Optional[torch.Generator] = None, return_logprobs: bool = False,
                   return_logits: bool = False, check_status: bool = True,
                   fused: Optional[bool] = None) -> LmHeadOutput:
    """One decode step's ``lm_head`` and sampling (one token per row).

    ``fused`` None picks the faster path for the shape (``fused_is_faster``):
    today always ``torch.nn.functional.linear`` followed by ``sample_tokens``,
    the reference's own two steps (``model.py:190,201``, ``sampling.py:16-61``).
    ``fused=True`` runs the fused kernels: rows they leave at ``FL_ROW_LIMIT``
    are sampled by ``fl_sample`` over the GEMM's logits, with the same
    uniforms, and batches above 64 rows run in groups of 64.  Any other row
    status raises ``SamplingError`` (unless ``check_status`` is off)."""
    B = hidden.size(0)
    if fused is None:
        fused = fused_is_faster(B, hidden.size(-1), weight.size(0))
    if not fused:
        if hidden.dim() != 2 or weight.dim() != 2 or hidden.size(1) != weight.size(1):
            raise ValueError(f"hidden [B, D] and weight [V, D] expected, got {tuple(hidden.shape)} and "
                             f"{tuple(weight.shape)}")
        if uniforms is None:
            uniforms = torch.rand(B, device=hidden.device, generator=generator)
        logits = torch.nn.functional.linear(hidden, weight)
        out = sample_tokens(logits, temperature=temperature, top_k=top_k, top_p=top_p, min_p=min_p,
                            repetition_penalty=1.0 if repetition_penalty is None else repetition_penalty,
                            history=history, softcap=softcap, uniforms=uniforms,
                            return_logprobs=return_logprobs, check_status=check_status)
        return LmHeadOutput(out.tokens, out.status, out.logprobs, logits if return_logits else None)
    if B > _lib.FL_LM_HEAD_MAX_BATCH:
        dev = hidden.device
        T, K = _per_row(temperature, B, torch.float32, dev, 1.0), _per_row(top_k, B, torch.int32, dev, 0)
        P, MP = _per_row(top_p, B, torch.float32, dev, 1.0), _per_row(min_p, B, torch.float32, dev, 0.0)
        RP = _per_row(repetition_penalty, B, torch.float32, dev, 1.0)
        hist, hlen, _ = _history_tensor(history, B, weight.size(0), dev)
        U = uniforms if uniforms is not None else torch.rand(B, device=dev, generator=generator)
        outs = []
        for s in range(0, B, _lib.FL_LM_HEAD_MAX_BATCH):
            e = min(B, s + _lib.FL_LM_HEAD_MAX_BATCH)
            outs.append(lm_head_sample(hidden[s:e], weight, temperature=T[s:e], top_k=K[s:e], top_p=P[s:e],
                                       min_p=MP[s:e], repetition_penalty=RP[s:e],
                                       history=None if hist is None else (hist[s:e], hlen[s:e]), softcap=softcap,
                                       uniforms=U[s:e], return_logprobs=return_logprobs,
                                       return_logits=return_logits, check_status=check_status, fused=True))
        cat = lambda xs: None if xs[0] is None else torch.cat(xs)  # noqa: E731
        return LmHeadOutput(cat([o.tokens for o in outs]), cat([o.status for o in outs]),
                            cat([o.logprobs for o in outs]), cat([o.logits for o in outs]))
    plan = LmHeadPlan(hidden, weight, temperature=temperature, top_k=top_k, top_p=top_p, min_p=min_p,
                      repetition_penalty=repetition_penalty, history=history, softcap=softcap, uniforms=uniforms,
                      generator=generator, return_logprobs=return_logprobs, return_logits=return_logits)
    plan.launch()
    out = plan.output
    limited = (out.status & _lib.FL_ROW_LIMIT) != 0
    if bool(limited.any()):
        rows = torch.nonzero(limited).flatten()
        logits = out.logits
        if logits is None:   # the GEMM again, with its logits output
            again = LmHeadPlan(hidden, weight, temperature=plan.T, top_k=plan.K, top_p=plan.P, min_p=plan.MP,
                               repetition_penalty=plan.RP, history=history, softcap=softcap, uniforms=plan.U,
                               return_logits=True)
            again.launch()
            logits = again.logits
        hist = None
        if plan.hist is not None:
            hist = (plan.hist.index_select(0, rows).contiguous(), plan.hist_len.index_select(0, rows).contiguous())
        sub = sample_tokens(logits.index_select(0, rows), temperature=plan.T[rows], top_k=plan.K[rows],
                            top_p=plan.P[rows], min_p=plan.MP[rows], repetition_penalty=plan.RP[rows], history=hist,
                            softcap=softcap, uniforms=plan.U[rows], return_logprobs=return_logprobs,
                            check_status=check_status)
        out.tokens.index_copy_(0, rows, sub.tokens)
        out.status.index_copy_(0, rows, sub.status)
        if out.logprobs is not None:
            out.logprobs.index_copy_(0, rows, sub.logprobs)
    if check_status:
        _raise_on_status(out.status)
    return out

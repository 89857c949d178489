"""Speculative-decoding verify on MI355X (reference
``src/forgeline/models/generation/speculative.py``).

``speculative_verify`` is the accept / resample / bonus step of
``SpeculativeGenerator.generate`` (``speculative.py:51-84``) for a batch of
sequences, in three launches: the filter kernel over the target rows (which
also draws the bonus token), the filter kernel over the draft rows, and the
verify kernel (one work-group per sequence).

Rules (as the reference): ``T = max(T, 1e-8)``; position i accepts draft d_i
iff ``u_accept[b, i] < min(1, p_i(d_i) / (q_i(d_i) + 1e-10))``; the first
rejection resamples from ``max(0, p_i - q_i)``; if every draft is accepted the
bonus token is drawn from target position K.  CONVENTIONS: the filters are the
full ``apply_sampling_filters`` set (the reference uses top-k only); draws are
inverse-CDF with caller uniforms -- descending filtered value for the bonus,
ascending vocabulary index for the residual.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Dict, Optional

import torch

from . import _lib
from ._lib import SpecArgs, check, lib, ptr
from .sampling import _DTYPES, _check_logits, describe_rows, sample_tokens


@dataclass
class SpecOutput:
    n_accepted: torch.Tensor        # int32 [B]
    tokens: torch.Tensor            # int64 [B, K+1]: accepted drafts, then the resampled / bonus token, -1 after
    ratio: Optional[torch.Tensor]   # float32 [B, K]: acceptance ratio of each examined draft (NaN if not examined)


def speculative_verify(target_logits: torch.Tensor, draft_logits: torch.Tensor, draft_ids: torch.Tensor, *,
                       temperature: float = 1.0, top_k: Optional[int] = None, top_p: Optional[float] = None,
                       min_p: Optional[float] = None, softcap: float = 0.0,
                       u_accept: Optional[torch.Tensor] = None, u_resample: Optional[torch.Tensor] = None,
                       generator: Optional[torch.Generator] = None, return_ratio: bool = True) -> SpecOutput:
    """Verify ``K`` drafted tokens for each of ``B`` sequences.

    target_logits [B, K+1, V] (positions of the K drafts plus the bonus
    position), draft_logits [B, K, V], draft_ids int64 [B, K]."""
    if target_logits.dim() != 3 or draft_logits.dim() != 3:
        raise ValueError("target_logits must be [B, K+1, V] and draft_logits [B, K, V]")
    B, K1, V = target_logits.shape
    K = K1 - 1
    if K < 1 or tuple(draft_logits.shape) != (B, K, V) or tuple(draft_ids.shape) != (B, K):
        raise ValueError(f"shape mismatch: target {tuple(target_logits.shape)}, draft {tuple(draft_logits.shape)}, "
                         f"draft_ids {tuple(draft_ids.shape)}")
    if target_logits.dtype != draft_logits.dtype:
        raise ValueError("target and draft logits must share a dtype")
    dev = target_logits.device
    T = max(float(temperature), 1e-8)
    if u_accept is None:
        u_accept = torch.rand(B, K, device=dev, generator=generator)
    if u_resample is None:
        u_resample = torch.rand(B, device=dev, generator=generator)
    u_accept = u_accept.to(device=dev, dtype=torch.float32).contiguous()
    u_resample = u_resample.to(device=dev, dtype=torch.float32).contiguous()
    filt = dict(temperature=T, top_k=top_k if (top_k is not None and top_k > 0) else 0,
                top_p=top_p if top_p is not None else 1.0, min_p=min_p if min_p is not None else 0.0,
                softcap=softcap)
    tgt = _check_logits(target_logits.reshape(B * K1, V))
    drf = _check_logits(draft_logits.reshape(B * K, V))
    t_out = sample_tokens(tgt, uniforms=u_resample.repeat_interleave(K1), return_desc=True, check_status=False,
                          **filt)
    d_desc, d_status = describe_rows(drf, **filt)
    n_acc = torch.empty(B, dtype=torch.int32, device=dev)
    tokens = torch.empty(B, K1, dtype=torch.int64, device=dev)
    ratio = torch.empty(B, K, dtype=torch.float32, device=dev) if return_ratio else None
    temps = torch.full((B,), T, dtype=torch.float32, device=dev)
    ids = draft_ids.to(device=dev, dtype=torch.int64).contiguous()
    a = SpecArgs()
    a.struct_size = ctypes.sizeof(SpecArgs)
    a.dtype = _DTYPES[target_logits.dtype]
    a.target, a.draft = tgt.data_ptr(), drf.data_ptr()
    a.batch, a.k, a.vocab, a.ld = B, K, V, V
    a.temperature, a.softcap = temps.data_ptr(), float(softcap or 0.0)
    a.target_desc, a.draft_desc = ptr(t_out.desc), ptr(d_desc)
    a.draft_ids, a.u_accept, a.u_resample = ids.data_ptr(), u_accept.data_ptr(), u_resample.data_ptr()
    a.bonus_token = t_out.tokens.data_ptr()
    a.out_n_accepted, a.out_tokens, a.out_ratio = n_acc.data_ptr(), tokens.data_ptr(), ptr(ratio)
    check(lib().fl_spec_verify(ctypes.byref(a), _lib.stream_handle(dev)), "fl_spec_verify")
    # keep the argument tensors alive until the kernels have consumed them
    _keep = (tgt, drf, t_out, d_desc, temps, ids, u_accept, u_resample)  # noqa: F841
    bad = (t_out.status != 0).view(B, K1).any(1) | (d_status != 0).view(B, K).any(1)
    if bool(bad.any()):
        from .sampling import SamplingError
        raise SamplingError(f"speculative verify: sequences {torch.nonzero(bad).flatten().tolist()[:8]} have "
                            "rows that cannot be sampled (NaN / +inf / fully masked logits)")
    return SpecOutput(n_acc, tokens, ratio)


class SpeculativeGenerator:
    """Draft ``k`` tokens with a small model, verify with the target in one
    pass (reference ``speculative.py:20-91``, batched over sequences).

    Models follow the reference protocol: ``model(idx) -> (logits [B, T, V], _)``,
    ``model.full_logits(idx) -> [B, T, V]`` and ``model.spec.block_size``."""

    def __init__(self, target_model, draft_model, k: int = 5):
        self.target = target_model
        self.draft = draft_model
        self.k = k
        self.stats: Dict[str, int] = {"proposed": 0, "accepted": 0}

    @torch.no_grad()
    def generate(self, idx: torch.Tensor, max_new_tokens: int, temperature: float = 1.0, top_k: Optional[int] = 50,
                 top_p: Optional[float] = None, generator: Optional[torch.Generator] = None) -> torch.Tensor:
        if idx.size(0) != 1:
            raise ValueError("SpeculativeGenerator.generate grows one sequence (use speculative_verify for batches)")
        T = max(temperature, 1e-8)
        generated = 0
        while generated < max_new_tokens:
            draft_tokens, draft_rows = [], []
            draft_idx = idx.clone()
            bs = self.draft.spec.block_size
            for _ in range(self.k):
                ctx = draft_idx if draft_idx.size(1) <= bs else draft_idx[:, -bs:]
                logits, _ = self.draft(ctx)
                row = logits[:, -1, :]
                tok = sample_tokens(row, temperature=T, top_k=top_k or 0, top_p=top_p or 1.0,
                                    uniforms=torch.rand(1, device=idx.device, generator=generator)).tokens.view(1, 1)
                draft_tokens.append(tok)
                draft_rows.append(row)
                draft_idx = torch.cat([draft_idx, tok], dim=1)
            verify_idx = torch.cat([idx] + draft_tokens, dim=1)
            tb = self.target.spec.block_size
            if verify_idx.size(1) > tb:
                verify_idx = verify_idx[:, -tb:]
            target_logits = self.target.full_logits(verify_idx)
            prompt_len = idx.size(1)
            offset = verify_idx.size(1) - (prompt_len + self.k)
            first = prompt_len - 1 + offset
            if first < 0 or first + self.k >= target_logits.size(1):
                break
            out = speculative_verify(target_logits[:, first:first + self.k + 1, :].contiguous(),
                                     torch.stack(draft_rows, dim=1), torch.cat(draft_tokens, dim=1),
                                     temperature=T, top_k=top_k, top_p=top_p, generator=generator)
            n = int(out.n_accepted[0])
            self.stats["proposed"] += min(n + 1, self.k)
            self.stats["accepted"] += n
            new = out.tokens[0, : n + 1]
            new = new[: max_new_tokens - generated]
            idx = torch.cat([idx, new.view(1, -1)], dim=1)
            generated += new.numel()
            if idx.size(1) >= tb:
                break
        return idx

    @property
    def acceptance_rate(self) -> float:
        return self.stats["accepted"] / max(self.stats["proposed"], 1)

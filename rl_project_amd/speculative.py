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
from .sampling import FL_FLAG_NO_SELECT, _DTYPES, _Call, _check_logits, sample_tokens


@dataclass
class SpecOutput:
    n_accepted: torch.Tensor        # int32 [B]
    tokens: torch.Tensor            # int64 [B, K+1]: accepted drafts, then the resampled / bonus token, -1 after
    ratio: Optional[torch.Tensor]   # float32 [B, K]: acceptance ratio of each examined draft (NaN if not examined)


class SpecPlan:
    """A prepared ``speculative_verify``: arguments and outputs are built once;
    each ``launch()`` enqueues the three kernels (target rows with the bonus
    draw, draft rows, verify) with no allocation and no host synchronisation.
    The logits, draft ids and uniforms are read at launch time, so a decode
    loop may overwrite them in place between launches.  ``sliced`` spreads the
    residual draw of each rejected sequence over several work-groups (with a
    workspace allocated here); ``sliced=False`` runs one work-group per
    sequence; ``no_alloc=True`` runs the sliced path on the library's static
    device scratch (``fl_spec_verify_static``: no workspace, at most 4096
    sequences, plans that launch at the same time on one GPU race).  All give
    identical results."""

    def __init__(self, target_logits: torch.Tensor, draft_logits: torch.Tensor, draft_ids: torch.Tensor, *,
                 temperature: float = 1.0, top_k: Optional[int] = None, top_p: Optional[float] = None,
                 min_p: Optional[float] = None, softcap: float = 0.0, u_accept: Optional[torch.Tensor] = None,
                 u_resample: Optional[torch.Tensor] = None, generator: Optional[torch.Generator] = None,
                 return_ratio: bool = True, sliced: bool = True, no_alloc: bool = False):
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
        self.B, self.K = B, K
        T = max(float(temperature), 1e-8)
        if u_accept is None:
            u_accept = torch.rand(B, K, device=dev, generator=generator)
        if u_resample is None:
            u_resample = torch.rand(B, device=dev, generator=generator)
        self.u_accept = u_accept.to(device=dev, dtype=torch.float32).contiguous()
        self.u_resample = u_resample.to(device=dev, dtype=torch.float32).contiguous()
        filt = dict(temperature=T, top_k=top_k if (top_k is not None and top_k > 0) else 0,
                    top_p=top_p if top_p is not None else 1.0, min_p=min_p if min_p is not None else 0.0,
                    softcap=softcap)
        tgt = _check_logits(target_logits.reshape(B * K1, V))
        drf = _check_logits(draft_logits.reshape(B * K, V))
        # the K+1 target rows of a sequence share its resample draw (read at
        # launch time, so in-place updates of u_resample reach the bonus draw)
        self._t = _Call(tgt, flags=0, want_desc=True, uniforms=self.u_resample, uniform_div=K1, **filt)
        self._d = _Call(drf, flags=FL_FLAG_NO_SELECT, want_desc=True, uniforms=None, **filt)
        self.n_accepted = torch.empty(B, dtype=torch.int32, device=dev)
        self.tokens = torch.empty(B, K1, dtype=torch.int64, device=dev)
        self.ratio = torch.empty(B, K, dtype=torch.float32, device=dev) if return_ratio else None
        self._temps = torch.full((B,), T, dtype=torch.float32, device=dev)
        self._ids = draft_ids.to(device=dev, dtype=torch.int64).contiguous()
        a = SpecArgs()
        a.struct_size = ctypes.sizeof(SpecArgs)
        a.dtype = _DTYPES[target_logits.dtype]
        a.target, a.draft = tgt.data_ptr(), drf.data_ptr()
        a.batch, a.k, a.vocab, a.ld = B, K, V, V
        a.temperature, a.softcap = self._temps.data_ptr(), float(softcap or 0.0)
        a.target_desc, a.draft_desc = ptr(self._t.desc), ptr(self._d.desc)
        a.draft_ids, a.u_accept, a.u_resample = self._ids.data_ptr(), self.u_accept.data_ptr(), self.u_resample.data_ptr()
        a.bonus_token = self._t.tokens.data_ptr()
        a.out_n_accepted, a.out_tokens, a.out_ratio = (self.n_accepted.data_ptr(), self.tokens.data_ptr(),
                                                       ptr(self.ratio))
        # scratch of the sliced residual draw (several work-groups per sequence)
        if no_alloc and B > _lib.FL_SPEC_STATIC_MAX_BATCH:
            raise ValueError(f"no_alloc verifies at most {_lib.FL_SPEC_STATIC_MAX_BATCH} sequences, not {B}")
        sliced = sliced and not no_alloc
        nbytes = ctypes.c_size_t(0)
        check(lib().fl_spec_workspace_bytes(B, ctypes.byref(nbytes)), "fl_spec_workspace_bytes")
        self._ws = torch.empty(max(int(nbytes.value), 8), dtype=torch.uint8, device=dev) if sliced else None
        a.workspace = ptr(self._ws)
        a.workspace_bytes = int(nbytes.value) if sliced else 0
        self._args = a
        self._argp = ctypes.byref(a)
        self._stream = _lib.stream_handle(dev)
        self._verify = lib().fl_spec_verify_static if no_alloc else lib().fl_spec_verify

    def launch(self) -> None:
        self._t.run()
        self._d.run()
        rc = self._verify(self._argp, self._stream)
        if rc:
            check(rc, self._verify.__name__)

    def status_ok(self) -> torch.Tensor:
        """bool [B]: every target and draft row of the sequence could be sampled."""
        B, K = self.B, self.K
        return ~((self._t.status != 0).view(B, K + 1).any(1) | (self._d.status != 0).view(B, K).any(1))

    @property
    def output(self) -> SpecOutput:
        return SpecOutput(self.n_accepted, self.tokens, self.ratio)


def speculative_verify(target_logits: torch.Tensor, draft_logits: torch.Tensor, draft_ids: torch.Tensor, *,
                       temperature: float = 1.0, top_k: Optional[int] = None, top_p: Optional[float] = None,
                       min_p: Optional[float] = None, softcap: float = 0.0,
                       u_accept: Optional[torch.Tensor] = None, u_resample: Optional[torch.Tensor] = None,
                       generator: Optional[torch.Generator] = None, return_ratio: bool = True) -> SpecOutput:
    """Verify ``K`` drafted tokens for each of ``B`` sequences.

    target_logits [B, K+1, V] (positions of the K drafts plus the bonus
    position), draft_logits [B, K, V], draft_ids int64 [B, K]."""
    plan = SpecPlan(target_logits, draft_logits, draft_ids, temperature=temperature, top_k=top_k, top_p=top_p,
                    min_p=min_p, softcap=softcap, u_accept=u_accept, u_resample=u_resample, generator=generator,
                    return_ratio=return_ratio)
    plan.launch()
    ok = plan.status_ok()
    if not bool(ok.all()):
        from .sampling import SamplingError
        raise SamplingError(f"speculative verify: sequences {torch.nonzero(~ok).flatten().tolist()[:8]} have "
                            "rows that cannot be sampled (NaN / +inf / fully masked logits)")
    return plan.output


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


class MTPSpeculativeGenerator:
    """Self-speculative decoding with the model's multi-token-prediction heads
    (reference ``speculative.py:94-158``), one sequence.

    Per round, as the reference:

    1. ``token_1`` is sampled from the main head.
    2. Each MTP head drafts the next token from the last hidden state and the
       previous token's embedding.
    3. ``token_1`` is appended.
    4. The drafts are verified against one forward pass over the extended
       sequence: accept while ``u < min(1, p/q)``; the first rejection
       resamples ``max(0, p − q)``. A round draws no bonus token.

    Filtering is the reference's ``_topk_filter(logits / T, top_k)``. Draws
    are the build's inverse CDF with uniforms from ``generator``; the draws
    and the verify run on the GPU path.  Model protocol: ``model(idx) ->
    (logits, _)`` setting ``model._last_hidden``; ``model.full_logits``,
    ``model.mtp_modules``, ``model.transformer.wte``, ``model.lm_head``,
    ``model.spec.block_size``."""

    def __init__(self, model):
        if getattr(model, "mtp_modules", None) is None or len(model.mtp_modules) == 0:
            raise ValueError("MTPSpeculativeGenerator requires a model with n_predict_tokens > 1")
        self.model = model
        self.n_drafts = len(model.mtp_modules)

    @torch.no_grad()
    def generate(self, idx: torch.Tensor, max_new_tokens: int = 200, temperature: float = 1.0,
                 top_k: Optional[int] = 50, generator: Optional[torch.Generator] = None) -> torch.Tensor:
        if idx.size(0) != 1:
            raise ValueError("MTPSpeculativeGenerator.generate grows one sequence")
        self.model.eval()
        T = max(float(temperature), 1e-8)
        k = top_k if (top_k is not None and top_k > 0) else 0
        dev = idx.device
        block = self.model.spec.block_size
        generated = 0

        def draw(row: torch.Tensor) -> torch.Tensor:
            u = torch.rand(1, device=dev, generator=generator)
            return sample_tokens(row, temperature=T, top_k=k, uniforms=u).tokens.view(1, 1)

        while generated < max_new_tokens:
            ctx = idx if idx.size(1) <= block else idx[:, -block:]
            logits, _ = self.model(ctx)
            last_h = self.model._last_hidden
            main_row = logits[:, -1, :]
            token_1 = draw(main_row)
            draft_tokens, draft_rows = [token_1], [main_row]
            prev_emb = self.model.transformer.wte(token_1)
            for mtp_mod in self.model.mtp_modules:
                h_mtp = mtp_mod(last_h[:, -1:, :], prev_emb)
                row = self.model.lm_head(h_mtp[:, -1, :])
                tok = draw(row)
                draft_tokens.append(tok)
                draft_rows.append(row)
                prev_emb = self.model.transformer.wte(tok)

            idx = torch.cat([idx, token_1], dim=1)
            generated += 1
            if generated >= max_new_tokens:
                break
            K = len(draft_tokens) - 1
            if K > 0:
                verify_idx = torch.cat([idx, torch.cat(draft_tokens[1:], dim=1)], dim=1)
                if verify_idx.size(1) > block:
                    verify_idx = verify_idx[:, -block:]
                verify_logits = self.model.full_logits(verify_idx)
                prompt_len = idx.size(1)
                offset = verify_idx.size(1) - (prompt_len + K)
                first = prompt_len - 1 + offset
                if first < 0 or first + K >= verify_logits.size(1):
                    # fewer verify positions than drafts (the context window cut them)
                    if idx.size(1) >= block:
                        break
                    continue
                # positions first .. first + K - 1 verify drafts 1..K; position
                # first + K would be the bonus, which this scheme does not draw
                out = speculative_verify(verify_logits[:, first:first + K + 1, :].contiguous(),
                                         torch.stack(draft_rows[1:], dim=1).to(verify_logits.dtype),
                                         torch.cat(draft_tokens[1:], dim=1), temperature=T, top_k=k or None,
                                         generator=generator)
                n = int(out.n_accepted[0])
                new = out.tokens[0, : (n if n == K else n + 1)]
                new = new[: max_new_tokens - generated]
                idx = torch.cat([idx, new.view(1, -1)], dim=1)
                generated += new.numel()
            if idx.size(1) >= block:
                break
        return idx

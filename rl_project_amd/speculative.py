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
from typing import Dict, List, Optional

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
    each ``launch()`` enqueues the kernels (target rows with the bonus draw,
    draft rows, verify) on the device's current stream with no allocation and
    no host synchronisation (so it may be captured in a graph).
    The logits, draft ids and uniforms are read at launch time, so a decode
    loop may overwrite them in place between launches.  ``sliced`` spreads the
    residual draw of each rejected sequence over several work-groups (with a
    workspace allocated here; with ``cache_residual`` the workspace also
    holds each rejected sequence's residual row, 4 bytes per vocabulary
    entry, so the second pass and the draw read it instead of recomputing
    both rows' probabilities); ``sliced=False`` runs one work-group per
    sequence; ``no_alloc=True`` runs the sliced path on the library's static
    device scratch (``fl_spec_verify_static``: no workspace, at most 4096
    sequences, plans that launch at the same time on one GPU race).  All give
    identical results."""

    def __init__(self, target_logits: torch.Tensor, draft_logits: torch.Tensor, draft_ids: torch.Tensor, *,
                 temperature: float = 1.0, top_k: Optional[int] = None, top_p: Optional[float] = None,
                 min_p: Optional[float] = None, softcap: float = 0.0, u_accept: Optional[torch.Tensor] = None,
                 u_resample: Optional[torch.Tensor] = None, generator: Optional[torch.Generator] = None,
                 return_ratio: bool = True, sliced: bool = True, no_alloc: bool = False,
                 cache_residual: bool = True):
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
        if cache_residual:
            check(lib().fl_spec_cache_workspace_bytes(B, V, ctypes.byref(nbytes)), "fl_spec_cache_workspace_bytes")
        else:
            check(lib().fl_spec_workspace_bytes(B, ctypes.byref(nbytes)), "fl_spec_workspace_bytes")
        self._ws = torch.empty(max(int(nbytes.value), 8), dtype=torch.uint8, device=dev) if sliced else None
        a.workspace = ptr(self._ws)
        a.workspace_bytes = int(nbytes.value) if sliced else 0
        self._args = a
        self._argp = ctypes.byref(a)
        self._dev = dev
        self._verify = lib().fl_spec_verify_static if no_alloc else lib().fl_spec_verify

    def launch(self) -> None:
        self._t.run()
        self._d.run()
        rc = self._verify(self._argp, _lib.stream_handle(self._dev))   # the current stream (graph capture records it)
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


def _as_sequences(idx) -> tuple:
    """(list of 1-D token tensors, whether the caller passed one [1, T] tensor)."""
    if isinstance(idx, torch.Tensor):
        if idx.dim() != 2:
            raise ValueError("idx must be [B, T] or a list of 1-D token tensors")
        return [idx[b] for b in range(idx.size(0))], idx.size(0) == 1
    seqs = [t.reshape(-1) for t in idx]
    if not seqs:
        raise ValueError("no sequences")
    return seqs, False


def _grouped(fn, ctxs: List[torch.Tensor]) -> List:
    """fn over the contexts, one call per group of equal length (a model
    forward takes [g, L] token ids); the results of row i of each call, in
    the order of ``ctxs``."""
    groups: Dict[int, List[int]] = {}
    for i, c in enumerate(ctxs):
        groups.setdefault(int(c.numel()), []).append(i)
    out: List = [None] * len(ctxs)
    for members in groups.values():
        res = fn(torch.stack([ctxs[i] for i in members]))
        for j, i in enumerate(members):
            out[i] = tuple(r[j] for r in res) if isinstance(res, tuple) else res[j]
    return out


def _result(seqs: List[torch.Tensor], single: bool):
    return seqs[0].view(1, -1) if single else [s.view(1, -1) for s in seqs]


class SpeculativeGenerator:
    """Draft ``k`` tokens with a small model, verify with the target in one
    pass (reference ``speculative.py:20-91``), for a batch of sequences.

    Each sequence follows the reference's one-sequence loop; the sequences of
    a batch advance together: per round, the draft model runs once per group
    of equal context length, each of the ``k`` draft draws is one sampler
    launch over every active sequence, the target runs once per length group,
    and one batched verify decides all of them (ragged acceptance: each
    sequence keeps its own accepted drafts plus its resampled or bonus token).

    ``idx``: a [1, T] tensor (returns [1, T'], as the reference), a [B, T]
    tensor or a list of 1-D prompts (returns a list of [1, T_b] tensors).
    ``trace``: a list that receives, per round, the active sequences and every
    draw and decision (for replay checks).  Models follow the reference
    protocol: ``model(idx) -> (logits [B, T, V], _)``,
    ``model.full_logits(idx) -> [B, T, V]`` and ``model.spec.block_size``."""

    def __init__(self, target_model, draft_model, k: int = 5):
        self.target = target_model
        self.draft = draft_model
        self.k = k
        self.stats: Dict[str, int] = {"proposed": 0, "accepted": 0}

    @torch.no_grad()
    def generate(self, idx, max_new_tokens: int, temperature: float = 1.0, top_k: Optional[int] = 50,
                 top_p: Optional[float] = None, generator: Optional[torch.Generator] = None,
                 trace: Optional[List[dict]] = None):
        seqs, single = _as_sequences(idx)
        dev = seqs[0].device
        T = max(temperature, 1e-8)
        K = self.k
        n = len(seqs)
        generated = [0] * n
        active = [max_new_tokens > 0] * n
        bs, tb = self.draft.spec.block_size, self.target.spec.block_size
        while True:
            act = [b for b in range(n) if active[b]]
            if not act:
                break
            # k draft draws, each one launch over the active sequences
            dctx = [seqs[b] for b in act]
            d_rows, d_toks, u_draft = [], [], []
            for _ in range(K):
                rows = torch.stack(_grouped(lambda x: self.draft(x)[0][:, -1, :],
                                            [c if c.numel() <= bs else c[-bs:] for c in dctx]))
                u = torch.rand(len(act), device=dev, generator=generator)
                tok = sample_tokens(rows, temperature=T, top_k=top_k or 0, top_p=top_p or 1.0, uniforms=u).tokens
                d_rows.append(rows)
                d_toks.append(tok)
                u_draft.append(u)
                dctx = [torch.cat([c, tok[i:i + 1].to(c.dtype)]) for i, c in enumerate(dctx)]
            drafts = torch.stack(d_toks, dim=1)                     # [A, K]
            vctx = [torch.cat([seqs[b], drafts[i].to(seqs[b].dtype)]) for i, b in enumerate(act)]
            vctx = [c if c.numel() <= tb else c[-tb:] for c in vctx]
            full = _grouped(lambda x: self.target.full_logits(x), vctx)
            # the verify positions of each sequence: prompt_len - 1 + offset ..
            # (+ K); the context is cut to the block size from the left
            rows_t, ok = [], []
            for i, b in enumerate(act):
                L = vctx[i].numel()
                first = seqs[b].numel() - 1 + (L - (seqs[b].numel() + K))
                if first < 0 or first + K >= full[i].size(0):
                    active[b] = False
                    continue
                rows_t.append(full[i][first:first + K + 1])
                ok.append(i)
            rec = {"seqs": act, "u_draft": torch.stack(u_draft, dim=1), "draft_tokens": drafts, "verified": ok}
            if ok:
                sel = torch.tensor(ok, device=dev)
                u_acc = torch.rand(len(ok), K, device=dev, generator=generator)
                u_res = torch.rand(len(ok), device=dev, generator=generator)
                out = speculative_verify(torch.stack(rows_t), torch.stack(d_rows, dim=1)[sel].contiguous(),
                                         drafts[sel].contiguous(), temperature=T, top_k=top_k, top_p=top_p,
                                         u_accept=u_acc, u_resample=u_res, return_ratio=False)
                n_acc = out.n_accepted.tolist()
                toks = out.tokens.tolist()
                rec.update(u_accept=u_acc, u_resample=u_res, n_accepted=n_acc, tokens=toks)
                for j, i in enumerate(ok):
                    b = act[i]
                    room = max_new_tokens - generated[b]
                    na = n_acc[j]
                    # drafts examined as the reference's loop does: up to the
                    # first rejection, or until the token budget is spent
                    self.stats["proposed"] += room if room <= na else min(na + 1, K)
                    self.stats["accepted"] += min(na, room)
                    new = toks[j][: na + 1][:room]
                    seqs[b] = torch.cat([seqs[b], torch.tensor(new, dtype=seqs[b].dtype, device=dev)])
                    generated[b] += len(new)
                    if generated[b] >= max_new_tokens or seqs[b].numel() >= tb:
                        active[b] = False
            if trace is not None:
                trace.append(rec)
        return _result(seqs, single)

    @property
    def acceptance_rate(self) -> float:
        return self.stats["accepted"] / max(self.stats["proposed"], 1)


class MTPSpeculativeGenerator:
    """Self-speculative decoding with the model's multi-token-prediction heads
    (reference ``speculative.py:94-158``), for a batch of sequences.

    Per round and sequence, as the reference:

    1. ``token_1`` is sampled from the main head.
    2. Each MTP head drafts the next token from the last hidden state and the
       previous token's embedding.
    3. ``token_1`` is appended.
    4. The drafts are verified against one forward pass over the extended
       sequence: accept while ``u < min(1, p/q)``; the first rejection
       resamples ``max(0, p − q)``. A round draws no bonus token.

    Batched: the main forward and the verify forward run once per group of
    equal context length, the MTP heads and every draw once over all active
    sequences, the verify in one launch (ragged acceptance).  Filtering is the
    reference's ``_topk_filter(logits / T, top_k)``. Draws are the build's
    inverse CDF with uniforms from ``generator``.  ``idx`` and ``trace`` as
    for ``SpeculativeGenerator``.  Model protocol: ``model(idx) ->
    (logits, _)`` setting ``model._last_hidden``; ``model.full_logits``,
    ``model.mtp_modules``, ``model.transformer.wte``, ``model.lm_head``,
    ``model.spec.block_size``."""

    def __init__(self, model):
        if getattr(model, "mtp_modules", None) is None or len(model.mtp_modules) == 0:
            raise ValueError("MTPSpeculativeGenerator requires a model with n_predict_tokens > 1")
        self.model = model
        self.n_drafts = len(model.mtp_modules)

    @torch.no_grad()
    def generate(self, idx, max_new_tokens: int = 200, temperature: float = 1.0, top_k: Optional[int] = 50,
                 generator: Optional[torch.Generator] = None, trace: Optional[List[dict]] = None):
        seqs, single = _as_sequences(idx)
        self.model.eval()
        T = max(float(temperature), 1e-8)
        k = top_k if (top_k is not None and top_k > 0) else 0
        dev = seqs[0].device
        block = self.model.spec.block_size
        n = len(seqs)
        generated = [0] * n
        active = [max_new_tokens > 0] * n

        def draw(rows: torch.Tensor, us: list) -> torch.Tensor:
            u = torch.rand(rows.size(0), device=dev, generator=generator)
            us.append(u)
            return sample_tokens(rows, temperature=T, top_k=k, uniforms=u).tokens

        def main_forward(x):
            logits, _ = self.model(x)
            return logits[:, -1, :], self.model._last_hidden[:, -1:, :]

        while True:
            act = [b for b in range(n) if active[b]]
            if not act:
                break
            res = _grouped(main_forward, [s if s.numel() <= block else s[-block:] for s in (seqs[b] for b in act)])
            main_rows = torch.stack([r[0] for r in res])
            last_h = torch.stack([r[1] for r in res])            # [A, 1, D]
            us: list = []
            token_1 = draw(main_rows, us)
            toks, rows = [token_1], [main_rows]
            prev_emb = self.model.transformer.wte(token_1.view(-1, 1))
            for mtp_mod in self.model.mtp_modules:
                h_mtp = mtp_mod(last_h, prev_emb)
                row = self.model.lm_head(h_mtp[:, -1, :])
                tok = draw(row, us)
                toks.append(tok)
                rows.append(row)
                prev_emb = self.model.transformer.wte(tok.view(-1, 1))
            drafts = torch.stack(toks[1:], dim=1)                  # [A, K]
            K = drafts.size(1)
            rec = {"seqs": act, "u_draft": torch.stack(us, dim=1), "token_1": token_1, "draft_tokens": drafts,
                   "verified": []}
            go = []
            for i, b in enumerate(act):
                seqs[b] = torch.cat([seqs[b], token_1[i:i + 1].to(seqs[b].dtype)])
                generated[b] += 1
                if generated[b] >= max_new_tokens:
                    active[b] = False
                else:
                    go.append(i)
            vctx = [torch.cat([seqs[act[i]], drafts[i].to(seqs[act[i]].dtype)]) for i in go]
            vctx = [c if c.numel() <= block else c[-block:] for c in vctx]
            full = _grouped(lambda x: self.model.full_logits(x), vctx)
            rows_t, ok = [], []
            for j, i in enumerate(go):
                L = vctx[j].numel()
                first = seqs[act[i]].numel() - 1 + (L - (seqs[act[i]].numel() + K))
                if first < 0 or first + K >= full[j].size(0):
                    continue   # fewer verify positions than drafts (the context window cut them)
                # positions first .. first + K - 1 verify drafts 1..K; position
                # first + K would be the bonus, which this scheme does not draw
                rows_t.append(full[j][first:first + K + 1])
                ok.append(i)
            rec["verified"] = ok
            if ok:
                sel = torch.tensor(ok, device=dev)
                d_rows = torch.stack(rows[1:], dim=1)[sel].to(rows_t[0].dtype).contiguous()
                u_acc = torch.rand(len(ok), K, device=dev, generator=generator)
                u_res = torch.rand(len(ok), device=dev, generator=generator)
                out = speculative_verify(torch.stack(rows_t), d_rows, drafts[sel].contiguous(), temperature=T,
                                         top_k=k or None, u_accept=u_acc, u_resample=u_res, return_ratio=False)
                n_acc = out.n_accepted.tolist()
                otoks = out.tokens.tolist()
                rec.update(u_accept=u_acc, u_resample=u_res, n_accepted=n_acc, tokens=otoks)
                for j, i in enumerate(ok):
                    b = act[i]
                    na = n_acc[j]
                    new = otoks[j][: (na if na == K else na + 1)][: max_new_tokens - generated[b]]
                    seqs[b] = torch.cat([seqs[b], torch.tensor(new, dtype=seqs[b].dtype, device=dev)])
                    generated[b] += len(new)
                    if generated[b] >= max_new_tokens:
                        active[b] = False
            for b in act:
                if seqs[b].numel() >= block:
                    active[b] = False
            if trace is not None:
                trace.append(rec)
        return _result(seqs, single)

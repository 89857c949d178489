"""Shared helpers of the parity tests: run the oracle on a workload and
classify the kernel's rows against it."""

from __future__ import annotations

from typing import List, Tuple

import numpy as np
import torch

from oracle import classify as C
from oracle import sampler_oracle as O


def unpack_mask(words: torch.Tensor, V: int) -> torch.Tensor:
    """int32 [B, ceil(V/32)] keep bit-mask -> bool [B, V] (CPU)."""
    w = words.cpu().to(torch.int64) & 0xFFFFFFFF
    bits = (w.unsqueeze(-1) >> torch.arange(32)) & 1
    return bits.reshape(w.size(0), -1)[:, :V].bool()


def row_params(w, b: int) -> O.RowParams:
    hist = [] if w.history is None else [int(v) for v in w.history[b].tolist() if v >= 0]
    stops = [] if w.stop_ids is None else [int(v) for v in w.stop_ids.tolist()]
    return O.RowParams(temperature=float(w.temperature[b]), top_k=int(w.top_k[b]), top_p=float(w.top_p[b]),
                       min_p=float(w.min_p[b]), repetition_penalty=float(w.repetition_penalty[b]), history=hist,
                       stop_ids=stops)


def oracle_rows(w) -> List[O.RowResult]:
    params = [row_params(w, b) for b in range(w.batch)]
    return O.sample_rows(w.logits.cpu(), params, w.uniforms.cpu().tolist(), softcap=w.softcap)


def classify_workload(w, got_tokens: torch.Tensor, got_keep: torch.Tensor = None,
                      ref: List[O.RowResult] = None,
                      got_values: torch.Tensor = None) -> Tuple[dict, List[C.RowVerdict]]:
    ref = ref if ref is not None else oracle_rows(w)
    x = w.logits.cpu()
    toks = got_tokens.cpu().tolist()
    verdicts = []
    for b in range(w.batch):
        rk = ~torch.isneginf(ref[b].filtered.float())
        gk = None if got_keep is None else got_keep[b]
        gv = None if got_values is None else got_values[b].cpu()
        verdicts.append(C.classify_row(x[b], row_params(w, b), float(w.uniforms[b]), rk, ref[b].token, gk, toks[b],
                                       softcap=w.softcap, got_values=gv))
    return C.summarise(verdicts), verdicts


# --------------------------------------------------------------------------
# Speculative verify
# --------------------------------------------------------------------------

def oracle_draft_sampler(temperature: float, top_p: float, top_k: int = 0):
    """Draft ids drawn from the filtered draft rows with the oracle's selection rule."""
    def draw(rows: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
        ids = []
        for r in range(rows.size(0)):
            filt = O.filter_logits(rows[r:r + 1], temperature, top_k or None, top_p, None)
            ids.append(O.select_token(filt[0], float(u[r]), temperature))
        return torch.tensor(ids, dtype=torch.int64)
    return draw


def spec_params(w) -> O.RowParams:
    return O.RowParams(temperature=w.temperature, top_k=int(getattr(w, "top_k", 0) or 0),
                       top_p=w.top_p if w.top_p is not None else 1.0)


def classify_spec(w, got_n: torch.Tensor, got_tokens: torch.Tensor):
    """Per sequence EXACT / NEAR / MISMATCH of a verify result against the
    oracle (``oracle.classify.classify_spec``)."""
    return C.classify_spec(w.target, w.draft, w.draft_ids, spec_params(w), w.u_accept, w.u_resample,
                           got_n.cpu().tolist(), got_tokens.cpu().tolist())

"""Shared helpers of the parity tests: run the oracle on a workload and
classify the kernel's rows against it."""

from __future__ import annotations

from typing import List, Tuple

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
                      ref: List[O.RowResult] = None) -> Tuple[dict, List[C.RowVerdict]]:
    ref = ref if ref is not None else oracle_rows(w)
    x = w.logits.cpu()
    toks = got_tokens.cpu().tolist()
    verdicts = []
    for b in range(w.batch):
        rk = ~torch.isneginf(ref[b].filtered.float())
        gk = None if got_keep is None else got_keep[b]
        verdicts.append(C.classify_row(x[b], row_params(w, b), float(w.uniforms[b]), rk, ref[b].token, gk, toks[b],
                                       softcap=w.softcap))
    return C.summarise(verdicts), verdicts

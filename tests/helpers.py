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


# --------------------------------------------------------------------------
# Speculative verify
# --------------------------------------------------------------------------

def oracle_draft_sampler(temperature: float, top_p: float):
    """Draft ids drawn from the filtered draft rows with the oracle's selection rule."""
    def draw(rows: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
        ids = []
        for r in range(rows.size(0)):
            filt = O.filter_logits(rows[r:r + 1], temperature, None, top_p, None)
            ids.append(O.select_token(filt[0], float(u[r]), temperature))
        return torch.tensor(ids, dtype=torch.int64)
    return draw


def _interval_hits(cum: torch.Tensor, pos: int, target: float, delta: float) -> bool:
    lo = 0.0 if pos == 0 else float(cum[pos - 1])
    hi = float(cum[pos])
    return hi > lo and lo <= target + delta and hi > target - delta


def classify_spec(w, got_n: torch.Tensor, got_tokens: torch.Tensor, rel: float = 1e-5):
    """Per sequence: EXACT, NEAR (the first difference is an accept decision
    with u within ``rel`` of the ratio, or a resampled / bonus token whose
    cumulative interval lies within ``rel`` of the draw) or MISMATCH."""
    p = O.RowParams(temperature=w.temperature, top_p=w.top_p)
    ref = O.speculative_verify(w.target, w.draft, w.draft_ids, p, w.u_accept, w.u_resample)
    B, K = w.draft_ids.shape
    gn = got_n.cpu().tolist()
    gt = got_tokens.cpu().tolist()
    out = []
    for b in range(B):
        r = ref[b]
        n = gn[b]
        toks = gt[b][:n + 1]
        if n == r.n_accepted and toks == r.tokens:
            out.append(("EXACT", 0.0))
            continue
        m = min(n, r.n_accepted)
        if n != r.n_accepted:
            ratio = r.accept_ratio[m]
            u = float(w.u_accept[b, m])
            margin = abs(u - ratio) / max(ratio, 1e-30)
            out.append(("NEAR" if margin <= rel else "MISMATCH", margin))
            continue
        u = float(np.float32(w.u_resample[b]))
        g = toks[-1]
        if n < K:   # residual at position n
            pt, _ = O.filtered_probs(w.target[b, n], p)
            pd, _ = O.filtered_probs(w.draft[b, n], p)
            rr = torch.clamp(pt - pd, min=0)
            rr = rr / (rr.sum() + 1e-10)
            wt = rr.double()
            if float(wt.sum()) <= 0.0:
                wt = pt.double()
            cum = torch.cumsum(wt, 0)
            tot = float(cum[-1])
            ok = _interval_hits(cum, g, u * tot, rel * tot)
        else:       # bonus from target position K
            _, filt = O.filtered_probs(w.target[b, K], p)
            probs = torch.softmax(filt, -1).double()
            order = O.selection_order(filt)
            cum = torch.cumsum(probs[order], 0)
            tot = float(cum[-1])
            pos = int((order == g).nonzero()[0]) if bool((order == g).any()) else 0
            ok = _interval_hits(cum, pos, u * tot, rel * tot)
        out.append(("NEAR" if ok else "MISMATCH", 0.0))
    kinds = [k for k, _ in out]
    summ = {k: kinds.count(k) for k in ("EXACT", "NEAR", "MISMATCH")}
    return summ, out, ref

"""Parity classifier: explain every difference between a candidate sampler's
result and the oracle's (test infrastructure only).

The contract (per row): the candidate's keep mask and token must equal the
oracle's, except for
  * TIE     -- inside a group of equal filtered values the two sides keep the
               same number of members but different ones (the reference's
               unstable sort leaves the order within a tie group open; the
               oracle and the kernel both keep the lowest indices);
  * NEAR    -- a decision whose outcome changes when the quantities it
               compares are perturbed by the oracle's own rounding error
               (relative ``rel``: PyTorch's CPU softmax is up to ~20 ulp from
               correctly rounded, float32 cumulative sums of bfloat16
               probabilities drift, tanh differs by an ulp); the margin is
               reported;
  * CONSEQ  -- a token difference that follows from an explained mask
               difference (the candidate's token is what the selection rule
               gives on the candidate's mask).
Anything else is MISMATCH.

Decision predicates re-evaluated here (reference ``sampling.py:36-61``):
top-k keeps y >= k-th largest; min-p keeps round(e r) >= round(round(r) min_p)
with r = 1/sum(e); top-p removes sorted position j when
round(round(C_j) - p_j) >= round(top_p); selection is the inverse CDF over
float64 cumulative probabilities.  ``round`` is the tensor dtype's rounding.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np
import torch
import torch.nn.functional as F

from . import sampler_oracle as O

REL = 1e-5


def _rn(x: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """float64 -> float32 -> dtype rounding, as float64."""
    t = torch.from_numpy(np.asarray(x, dtype=np.float64)).to(torch.float32)
    if dtype != torch.float32:
        t = t.to(dtype)
    return t.double().numpy()


@dataclass
class RowVerdict:
    kind: str                      # EXACT, TIE, NEAR, CONSEQ, MISMATCH
    details: List[str] = field(default_factory=list)
    margin: float = 0.0

    @property
    def ok(self) -> bool:
        return self.kind != "MISMATCH"


def _perturbed(fn, vals, rel) -> bool:
    """True when fn(*vals) changes under relative perturbations of each input."""
    base = fn(*vals)
    for i in range(len(vals)):
        for s in (-1.0, 1.0):
            v = list(vals)
            v[i] = v[i] * (1.0 + s * rel)
            if fn(*v) != base:
                return True
    return False


def classify_row(x: torch.Tensor, p: O.RowParams, u: float, ref_keep: torch.Tensor, ref_tok: int,
                 got_keep: Optional[torch.Tensor], got_tok: Optional[int], softcap: float = 0.0,
                 rel: float = REL) -> RowVerdict:
    """Classify one row.  ``x``: the input row [V]; ``ref_keep``/``got_keep``:
    bool [V] keep masks (``got_keep`` may be None to check the token only)."""
    dt = x.dtype
    same_mask = got_keep is None or bool(torch.equal(ref_keep, got_keep))
    if same_mask and (got_tok is None or got_tok == ref_tok):
        return RowVerdict("EXACT")
    hist = p.history if p.repetition_penalty != 1.0 else None
    y_t = O.pre_filter_values(x[None], p.temperature, p.repetition_penalty, hist, softcap)[0]
    y = y_t.double().numpy()
    V = y.size
    verdict = RowVerdict("TIE")
    margins: List[float] = []

    if not same_mask:
        diff = np.nonzero((ref_keep != got_keep).numpy())[0]
        # survivors of top-k and min-p as the oracle computes them
        stage = y_t[None].clone()
        stage = O._top_k(stage, p.top_k or None)
        kth = float(torch.topk(y_t, min(p.top_k, V)).values[-1]) if p.top_k and p.top_k > 0 else -np.inf
        pre_minp = stage.clone()
        stage = O._min_p(stage, p.min_p or None)
        surv = ~np.isneginf(stage[0].double().numpy())
        for v in np.unique(y[diff]):
            grp = np.nonzero(y == v)[0]
            nr, ng = int(ref_keep[grp].sum()), int(got_keep[grp].sum())
            if nr == ng:
                verdict.details.append(f"tie group y={v:.9g} n={grp.size} kept={nr}")
                continue
            explained = False
            # top-k boundary: exact on values; only soft-capped values can flip
            if p.top_k and softcap > 0 and abs(v - kth) <= 4 * np.spacing(np.float32(abs(kth))):
                explained = True
                margins.append(abs(v - kth) / max(abs(kth), 1e-30))
                verdict.details.append(f"near top-k (soft-cap) y={v:.9g} kth={kth:.9g}")
            # min-p boundary
            if not explained and p.min_p and p.min_p > 0:
                probs = F.softmax(pre_minp, dim=-1)[0].double().numpy()
                e = np.exp(v - y.max())
                S = np.exp(pre_minp[0].double().numpy() - y.max())
                S = S[np.isfinite(pre_minp[0].double().numpy())].sum()
                r = 1.0 / S

                mp = np.float32(p.min_p)  # torch multiplies by the Python scalar in float32

                def keep_minp(e_, r_):
                    return _rn(e_ * r_, dt) >= _rn(_rn(r_, dt) * mp, dt)
                # the same test on the oracle's own softmax output, whose
                # rounding may differ from the exact value's by one unit
                keep_or = bool(probs[grp[0]] >= _rn(probs.max() * mp, dt))
                if _perturbed(lambda a, b: bool(keep_minp(a, b)), [e, r], rel) or keep_or != bool(keep_minp(e, r)):
                    explained = True
                    margins.append(abs(e * r - float(_rn(_rn(r, dt) * mp, dt))) / (e * r))
                    verdict.details.append(f"near min-p y={v:.9g}")
                del probs
            # top-p boundary
            if not explained and p.top_p is not None and 0 < p.top_p < 1:
                vals = torch.from_numpy(np.where(surv, y, -np.inf)).to(dt)
                srt, order = torch.sort(vals, descending=True, stable=True)
                ps = F.softmax(srt, dim=-1).double().numpy()
                C = np.cumsum(ps)
                t = float(_rn(np.float64(p.top_p), dt))
                pos = np.nonzero(np.isin(order.numpy(), grp))[0]
                # A probability may come out one unit of the dtype apart on
                # the two sides: where the oracle's own softmax rounds away from
                # the correctly rounded value (torch's vectorised float32
                # softmax on the CPU is up to ~5e-5 relative off), or where the
                # exact value sits within `rel` of a rounding midpoint.  A
                # whole group of such members moves the cumulative sums after
                # it by the group's size in units.
                p64 = F.softmax(srt.double(), dim=-1).numpy()
                amb = np.maximum(np.abs(_rn(p64 * (1.0 + rel), dt) - _rn(p64 * (1.0 - rel), dt)),
                                 np.abs(ps - _rn(p64, dt)))
                # for 16-bit rows the reference accumulates the cumulative sums
                # sequentially in float32 (float32 rows: in float64); the
                # drift from the exact sums adds to the doubt
                drift = 0.0
                if dt != torch.float32:
                    drift = np.abs(np.cumsum(ps.astype(np.float32), dtype=np.float32).astype(np.float64) - C)
                U = np.cumsum(amb) - amb + drift

                def removed(c, pp):
                    return bool(_rn(_rn(c, dt) - pp, dt) >= t)
                for j in pos:
                    if _perturbed(removed, [C[j], ps[j]], rel) or removed(C[j] - U[j], ps[j]) != removed(C[j] + U[j], ps[j]):
                        explained = True
                        margins.append(abs(C[j] - ps[j] - p.top_p) / max(p.top_p, 1e-30))
                        verdict.details.append(f"near top-p y={v:.9g} excl={C[j] - ps[j]:.9g} top_p={p.top_p}")
                        break
            if not explained:
                verdict.kind = "MISMATCH"
                verdict.details.append(f"mask group y={v:.9g} n={grp.size}: ref kept {nr}, got kept {ng}")
        if verdict.kind != "MISMATCH":
            verdict.kind = "NEAR" if margins else "TIE"

    if got_tok is not None and got_tok != ref_tok and verdict.kind != "MISMATCH":
        keep = (got_keep if got_keep is not None else ref_keep).numpy()
        filt = torch.from_numpy(np.where(keep, y, -np.inf)).to(dt)
        expect = O.select_token(filt, u, p.temperature)
        if expect == got_tok and not same_mask:
            verdict.kind = "CONSEQ" if verdict.kind == "TIE" else verdict.kind
            verdict.details.append(f"token {got_tok} follows from the mask difference")
        else:
            probs = F.softmax(filt, dim=-1)
            if p.temperature <= 0:
                pr = probs.double().numpy()
                m = abs(pr[got_tok] - pr[expect]) / max(pr[expect], 1e-300)
                ok = pr[got_tok] > 0 and m <= rel * 4
            else:
                order = O.selection_order(filt).numpy()
                pr = probs.double().numpy()[order]
                C = np.cumsum(pr)
                target = np.float64(np.float32(u)) * C[-1]
                jg = int(np.nonzero(order == got_tok)[0][0])
                lo_c = C[jg - 1] if jg > 0 else 0.0
                hi_c = C[jg]
                m = 0.0 if lo_c <= target < hi_c else min(abs(target - lo_c), abs(target - hi_c)) / C[-1]
                ok = m <= rel
            if ok:
                verdict.kind = "NEAR"
                margins.append(m)
                verdict.details.append(f"near selection: token {got_tok} vs {ref_tok}, margin {m:.3g}")
            else:
                verdict.kind = "MISMATCH"
                verdict.details.append(f"token {got_tok} vs oracle {ref_tok} (expected {expect} on got mask)")
    elif got_tok is not None and got_tok != ref_tok:
        verdict.details.append(f"token {got_tok} vs oracle {ref_tok}")
    verdict.margin = max(margins) if margins else 0.0
    return verdict


def summarise(verdicts: List[RowVerdict]) -> dict:
    out = {k: 0 for k in ("EXACT", "TIE", "NEAR", "CONSEQ", "MISMATCH")}
    for v in verdicts:
        out[v.kind] += 1
    out["max_margin"] = max([v.margin for v in verdicts] + [0.0])
    return out

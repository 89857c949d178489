"""Parity classifier: explain every difference between a candidate sampler's
result and the oracle's (test infrastructure only).

The contract (per row): the candidate's keep mask and token must equal the
oracle's, except for
  * TIE     -- inside a group of equal filtered values the two sides keep the
               same number of members but different ones (the reference's
               unstable sort leaves the order within a tie group open; the
               oracle and the kernel both keep the lowest indices);
  * NEAR    -- a decision that the rounding doubt between the two
               computations leaves open; the doubt is computed, not assumed:
                 min-p      the float64 probabilities perturbed by the
                            kernels' own rounding (``RK`` relative) and the
                            oracle's own softmax output;
                 top-p      the gap between the reference's cumulative sums
                            (sequential float32 for 16-bit rows, float64
                            rounded to float32 for float32 rows) and exact
                            sums of correctly rounded probabilities, plus
                            every earlier probability whose rounding is open;
                            the group's kept count must lie in the range this
                            leaves (``_top_p_count_range``), on the oracle's
                            survivors or on another survivor set a correct
                            kernel may reach: open min-p decisions
                            (``_min_p_survivor_sets``), or on a soft-capped
                            row the values within 4 units of the K-th value
                            (``_softcap_top_k_survivor_sets``);
                 selection  the draw must fall within the doubt of the
                            chosen token's cumulative interval
                            (``selection_near``); on a soft-capped row, on the
                            kernel's own filtered values when they are the
                            oracle's within a few units of the dtype
                            (``_softcap_selection_near``); greedy picks must be able to
                            win the first-index argmax under ``RK``
                            (``greedy_near``);
                 soft-cap   a soft-capped row's mask and draw judged as the
                            oracle's filters and selection on the kernel's
                            own unfiltered values, when those are the
                            oracle's within a few units of the dtype
                            (``_softcap_on_kernel_values``);
                 speculative  accept ratios and residual / bonus draws
                            with the oracle's filtered rows and, where a
                            row's top-p cut is open (``_top_p_count_range``),
                            with each other allowed kept count
                            (``_top_p_alternatives``);
               the distance from the boundary is reported;
  * CONSEQ  -- a token difference that follows from an explained mask
               difference (the candidate's token is what the selection rule
               gives on the candidate's mask).
Anything else is MISMATCH.  ``tests/test_classify.py`` plants mistakes
(an extra token, a top-p cut moved by one value group, a token one position
off in the inverse CDF, a wrong greedy tie-break, wrong accept / residual /
bonus draws, tokens next to a bonus draw at an open top-p cut) and requires
MISMATCH for each.

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

REL = 1e-5   # kept for callers that pass rel; the decisions use computed doubts

# Relative rounding doubt of one probability as the kernels compute it
# (exp, one reciprocal and one product in float32: a few ulp), with a margin.
RK = 1e-6


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


def _top_p_count_range(y: np.ndarray, surv: np.ndarray, grp: np.ndarray, top_p: float, dt) -> tuple:
    """Range of kept counts of the value group ``grp`` that the top-p rule
    (``sampling.py:45-51``: sorted position j is removed when
    ``round(round(C_j) - p_j) >= round(top_p)``) allows under rounding doubt,
    and the exclusive mass at the group's first member.

    The reference's cumulative sums are the oracle's: sequential float32
    sums of the dtype-rounded probabilities for 16-bit rows, float64 sums
    rounded to float32 for float32 rows.  A kernel sums correctly rounded
    probabilities exactly, up to its own rounding (relative ``RK``).  The
    doubt at position j is the gap between the two sums there plus every
    earlier probability whose rounding is open.  Members whose decision holds
    at both ends of the doubt are certain; kept members form a prefix of the
    group in sorted order, so the count lies between the certain kept prefix
    and the members not certainly removed."""
    vals = torch.from_numpy(np.where(surv, y, -np.inf)).to(dt)
    srt, order = torch.sort(vals, descending=True, stable=True)
    ps = F.softmax(srt, dim=-1).double().numpy()
    p64 = F.softmax(srt.double(), dim=-1).numpy()
    t = float(_rn(np.float64(top_p), dt))
    if dt == torch.float32:
        c_ref = _rn(np.cumsum(ps), dt)
    else:
        c_ref = np.cumsum(ps.astype(np.float32), dtype=np.float32).astype(np.float64)
    pk = _rn(p64, dt)
    amb = np.abs(_rn(p64 * (1.0 + RK), dt) - _rn(p64 * (1.0 - RK), dt)) + np.abs(ps - pk)
    c_k = np.cumsum(pk)
    U = np.abs(c_ref - c_k) + np.cumsum(amb) + 1e-12
    pos = np.nonzero(np.isin(order.numpy(), grp))[0]

    # the removal test of every member at the 9 corners of its doubt
    s1, s2 = np.repeat([-1.0, 0.0, 1.0], 3)[:, None], np.tile([-1.0, 0.0, 1.0], 3)[:, None]
    c = c_ref[pos][None, :] + s1 * U[pos][None, :]
    pp = ps[pos][None, :] + s2 * amb[pos][None, :]
    rem = _rn(_rn(c, dt) - pp, dt) >= t
    some, every = rem.any(axis=0), rem.all(axis=0)
    # kept members form a prefix: certain kept up to the first member that
    # may be removed, possibly kept up to the first one certainly removed
    lo_n = int(np.argmax(some)) if some.any() else int(pos.size)
    hi_n = int(np.argmax(every)) if every.any() else int(pos.size)
    j0 = pos[0] if pos.size else 0
    return lo_n, hi_n, float(c_ref[j0] - ps[j0]) if pos.size else 0.0


def _softcap_top_k_survivor_sets(y: np.ndarray, top_k: int, cap: int = 16) -> List[np.ndarray]:
    """Top-k survivor sets (bool [V]) a correct kernel may reach on a
    soft-capped row: its soft-capped values may lie up to 4 units of the
    last place from the oracle's (the bound the top-k boundary rule above
    uses), so the elements within that band of the K-th value may fall on
    either side of the kernel's own K-th value (``sampling.py:36-38`` keeps
    every value >= it).  Their masses differ by parts in 10^6, so a top-p cut
    depends on how many of them survive, not on which: one set per count,
    from the fewest that still give K survivors to all of them."""
    V = y.size
    k = min(int(top_k), V)
    srt = np.sort(y)[::-1]
    kth = float(srt[k - 1])
    band = 4 * np.spacing(np.float32(abs(kth)))
    core = y > kth + band
    doubt = np.nonzero(np.abs(y - kth) <= band)[0]
    doubt = doubt[np.argsort(-y[doubt], kind="stable")]
    n_core = int(core.sum())
    sets = []
    for c in range(max(0, k - n_core), doubt.size + 1):
        s = core.copy()
        s[doubt[:c]] = True
        sets.append(s)
        if len(sets) >= cap:
            break
    return sets


def _min_p_survivor_sets(pre_minp: np.ndarray, probs: np.ndarray, min_p: float, dt, cap: int = 8) -> List[np.ndarray]:
    """The min-p survivor sets (bool [V]) that the rounding doubt leaves open
    (``sampling.py:40-43``): the oracle's first, then the others.

    min-p keeps ``round(e r) >= round(round(r) min_p)`` with ``r = 1/sum(e)``
    over the top-k survivors ``pre_minp`` (float64, -inf where removed); the
    test is monotone in ``e``, so the survivors are a prefix of the distinct
    values in descending order.  A value's decision is open when it flips
    under the kernels' relative rounding ``RK`` of ``e`` or ``r``, or when the
    oracle's own softmax output (``probs``) decides it otherwise.  Every prefix
    whose boundary lies in the band of open values is a survivor set a
    correct kernel may reach; a top-p cut is then judged on the set the kernel
    used, since its cumulative sums run over those survivors."""
    fin = np.isfinite(pre_minp)
    vals = np.unique(pre_minp[fin])[::-1]
    M = float(vals[0])
    e = np.exp(vals - M)
    S = float(np.exp(pre_minp[fin] - M).sum())
    r = 1.0 / S
    mp = np.float32(min_p)

    def keep(e_, r_):
        return _rn(e_ * r_, dt) >= _rn(_rn(np.array([r_]), dt) * mp, dt)[0]

    exact = keep(e, r)
    flips = np.zeros(vals.size, dtype=bool)
    for fe, fr in ((1 - 4 * RK, 1.0), (1 + 4 * RK, 1.0), (1.0, 1 - 4 * RK), (1.0, 1 + 4 * RK)):
        flips |= keep(e * fe, r * fr) != exact
    # the oracle's decision per distinct value: its softmax output at a member
    first = {}
    idx = np.nonzero(fin)[0]
    for i in idx[np.unique(pre_minp[idx], return_index=True)[1]]:
        first[pre_minp[i]] = i
    thr_or = _rn(np.array([probs.max() * mp]), dt)[0]
    oracle = np.array([probs[first[v]] >= thr_or for v in vals])
    open_ = flips | (oracle != exact)
    n_sure = int(np.argmax(~(exact & ~open_))) if not (exact & ~open_).all() else vals.size
    n_max = int(np.nonzero(exact | open_)[0].max()) + 1 if (exact | open_).any() else 0
    n_or = int(oracle.sum())
    sets = [fin & (pre_minp >= vals[n_or - 1])] if n_or > 0 else [np.zeros_like(fin)]
    for n in range(max(n_sure, 1), min(n_max, n_sure + cap) + 1):
        if n != n_or:
            sets.append(fin & (pre_minp >= vals[n - 1]))
    return sets


def classify_row(x: torch.Tensor, p: O.RowParams, u: float, ref_keep: torch.Tensor, ref_tok: int,
                 got_keep: Optional[torch.Tensor], got_tok: Optional[int], softcap: float = 0.0,
                 rel: float = REL, got_values: Optional[torch.Tensor] = None,
                 got_all_values: Optional[torch.Tensor] = None) -> RowVerdict:
    """Classify one row.  ``x``: the input row [V]; ``ref_keep``/``got_keep``:
    bool [V] keep masks (``got_keep`` may be None to check the token only).
    ``got_values``: the kernel's filtered values of the row (-inf outside its
    mask), used only for soft-capped rows (see ``_softcap_selection_near``).
    ``got_all_values``: the kernel's unfiltered values of the row (soft-cap,
    penalty and temperature applied, nothing removed), used only for
    soft-capped rows (see ``_softcap_on_kernel_values``)."""
    same_mask = got_keep is None or bool(torch.equal(ref_keep, got_keep))
    if same_mask and (got_tok is None or got_tok == ref_tok):
        return RowVerdict("EXACT")
    hist = p.history if p.repetition_penalty != 1.0 else None
    y_t = O.pre_filter_values(x[None], p.temperature, p.repetition_penalty, hist, softcap)[0]
    verdict = _classify_on(y_t, p, u, ref_keep, ref_tok, got_keep, got_tok, softcap, got_values)
    if verdict.kind == "MISMATCH" and softcap > 0 and got_all_values is not None:
        alt = _softcap_on_kernel_values(y_t, got_all_values, p, u, got_keep, got_tok, softcap, got_values)
        if alt is not None:
            return alt
    return verdict


def _classify_on(y_t: torch.Tensor, p: O.RowParams, u: float, ref_keep: torch.Tensor, ref_tok: int,
                 got_keep: Optional[torch.Tensor], got_tok: Optional[int], softcap: float,
                 got_values: Optional[torch.Tensor]) -> RowVerdict:
    """``classify_row`` on given pre-filter values ``y_t`` [V] (the values the
    filters compare), with ``ref_keep`` / ``ref_tok`` the oracle's result on
    them."""
    dt = y_t.dtype
    same_mask = got_keep is None or bool(torch.equal(ref_keep, got_keep))
    if same_mask and (got_tok is None or got_tok == ref_tok):
        return RowVerdict("EXACT")
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
        minp_sets = None
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
                if _perturbed(lambda a, b: bool(keep_minp(a, b)), [e, r], 4 * RK) or keep_or != bool(keep_minp(e, r)):
                    explained = True
                    margins.append(abs(e * r - float(_rn(_rn(r, dt) * mp, dt))) / (e * r))
                    verdict.details.append(f"near min-p y={v:.9g}")
                del probs
            # top-p boundary: the group's kept count must lie in the range
            # that the rounding doubt of the cumulative sums leaves open
            # (on every min-p survivor set the rounding doubt allows: the
            # kernel's cumulative sums run over the survivors it kept)
            if not explained and p.top_p is not None and 0 < p.top_p < 1:
                sets = [surv]
                if p.min_p and p.min_p > 0:
                    if minp_sets is None:
                        pm = pre_minp[0].double().numpy()
                        minp_sets = _min_p_survivor_sets(pm, F.softmax(pre_minp, dim=-1)[0].double().numpy(),
                                                         p.min_p, dt)[1:]
                    sets = sets + minp_sets
                n_minp = len(sets)
                if softcap > 0 and p.top_k and 0 < p.top_k < V and not (p.min_p and p.min_p > 0):
                    # (a top-p cut runs over the top-k survivors the kernel's
                    # own soft-capped values leave)
                    sets = sets + _softcap_top_k_survivor_sets(y, p.top_k)
                for k, s in enumerate(sets):
                    lo_n, hi_n, excl = _top_p_count_range(y, s, grp, p.top_p, dt)
                    if lo_n <= ng <= hi_n:
                        explained = True
                        margins.append(abs(excl - p.top_p) / max(p.top_p, 1e-30))
                        verdict.details.append(f"near top-p y={v:.9g} excl={excl:.9g} top_p={p.top_p} "
                                               f"kept {ng} in [{lo_n}, {hi_n}]" +
                                               (f" (min-p survivors: open set {k})" if 0 < k < n_minp else "") +
                                               (f" (soft-cap top-k survivors: set {k - n_minp})" if k >= n_minp
                                                else ""))
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
            if p.temperature <= 0:
                ok, m = greedy_near(filt, got_tok, expect)
            else:
                ok, m = selection_near(filt, u, got_tok)
            if ok:
                verdict.kind = "NEAR"
                margins.append(m)
                verdict.details.append(f"near selection: token {got_tok} vs {ref_tok}, margin {m:.3g}")
            elif softcap > 0 and p.temperature > 0 and got_values is not None and \
                    _softcap_selection_near(y, got_values, keep, u, got_tok, dt):
                verdict.kind = "NEAR"
                margins.append(m)
                verdict.details.append(f"near selection on the kernel's soft-capped values: token {got_tok} vs "
                                       f"{ref_tok}, distance {m:.3g} on the oracle's")
            else:
                verdict.kind = "MISMATCH"
                verdict.details.append(f"token {got_tok} vs oracle {ref_tok} (expected {expect} on got mask), "
                                       f"distance {m:.3g}")
    elif got_tok is not None and got_tok != ref_tok:
        verdict.details.append(f"token {got_tok} vs oracle {ref_tok}")
    verdict.margin = max(margins) if margins else 0.0
    return verdict




def _cdf_doubt(w_oracle: np.ndarray, w_exact: np.ndarray, dt) -> tuple:
    """Normalised inclusive cumulative sums of the oracle's weights and, per
    position, how far a kernel's cumulative may lie from them.

    ``w_oracle``: the weights the oracle accumulates (its dtype-rounded
    probabilities); ``w_exact``: the float64 weights.  A kernel computes each
    weight correctly rounded to the dtype up to its own rounding (relative
    ``RK``) and accumulates exactly, so its normalised cumulative differs from
    the oracle's by the measured gap between the oracle's cumulative and the
    correctly rounded one, plus the weights whose rounding is open under
    ``RK``.  Both are summed position by position: the doubt grows only where
    the two computations can actually differ."""
    wk = _rn(w_exact, dt)
    amb = np.abs(_rn(w_exact * (1.0 + RK), dt) - _rn(w_exact * (1.0 - RK), dt))
    so, sk = float(w_oracle.sum()), float(wk.sum())
    c_or = np.cumsum(w_oracle) / so
    c_k = np.cumsum(wk) / sk
    doubt = np.abs(c_or - c_k) + np.cumsum(amb) / sk + 1e-12
    return c_or, doubt


def selection_near(filt: torch.Tensor, u: float, got_tok: int) -> tuple:
    """(acceptable, distance) for an inverse-CDF draw that picked ``got_tok``
    on the filtered row ``filt``: acceptable when the draw ``u`` lies within
    the rounding doubt of ``got_tok``'s cumulative interval.  The distance is
    how far ``u`` lies outside the interval (0 inside)."""
    dt = filt.dtype
    order = O.selection_order(filt).numpy()
    ps = F.softmax(filt, dim=-1).double().numpy()[order]
    p64 = F.softmax(filt.double(), dim=-1).numpy()[order]
    pos = np.nonzero(order == got_tok)[0]
    if pos.size == 0 or p64[pos[0]] <= 0.0:
        return False, float("inf")
    j = int(pos[0])
    c, d = _cdf_doubt(ps, p64, dt)
    t = float(np.float64(np.float32(u)))
    lo, hi = (c[j - 1], d[j - 1]) if j > 0 else (0.0, 0.0), (c[j], d[j])
    dist = max(0.0, lo[0] - t, t - hi[0])
    return bool(lo[0] - lo[1] <= t < hi[0] + hi[1]), dist


SOFTCAP_ULPS = {torch.float32: 8, torch.bfloat16: 2, torch.float16: 2}


def _softcap_on_kernel_values(y_t: torch.Tensor, got_all_values: torch.Tensor, p: O.RowParams, u: float,
                              got_keep: Optional[torch.Tensor], got_tok: Optional[int], softcap: float,
                              got_values: Optional[torch.Tensor]) -> Optional[RowVerdict]:
    """A soft-capped row whose mask or draw differs from the oracle's because
    the kernel's tanh rounded values to a neighbouring representable number:
    the soft-cap flattens large values into a few value groups at and next
    to the cap, so one unit moves an element from one group to the next,
    across a top-p or min-p cut or past the draw.  NEAR when the kernel's
    unfiltered values ``got_all_values`` are the oracle's ``y_t`` within
    ``SOFTCAP_ULPS`` units of the dtype (the same elements -inf) and the
    kernel's mask and token are what the oracle's own filters and selection
    give on those values, up to TIE / NEAR / CONSEQ; None otherwise."""
    dt = y_t.dtype
    g = got_all_values.to(dt)
    yn, gn = y_t.double().numpy(), g.double().numpy()
    fin = np.isfinite(yn)
    if not np.array_equal(fin, np.isfinite(gn)) or not np.array_equal(yn[~fin], gn[~fin]):
        return None
    mant = {torch.float32: 23, torch.bfloat16: 7, torch.float16: 10}[dt]
    yk, gk = yn[fin], gn[fin]
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(yk), torch.finfo(dt).tiny))) - mant)
    units = np.abs(gk - yk) / ulp
    if yk.size and float(units.max()) > SOFTCAP_ULPS[dt]:
        return None
    stage = g[None].clone()
    stage = O._top_k(stage, p.top_k or None)
    stage = O._min_p(stage, p.min_p or None)
    stage = O._top_p(stage, p.top_p, True)
    keep = ~torch.isneginf(stage[0])
    tok = O.select_token(stage[0], u, p.temperature)
    v = _classify_on(g, p, u, keep, tok, got_keep, got_tok, softcap, got_values)
    if v.kind == "MISMATCH":
        return None
    moved = int(np.count_nonzero(units))
    out = RowVerdict("NEAR", details=[f"on the kernel's soft-capped values ({moved} differ from the oracle's, "
                                      f"at most {float(units.max()) if yk.size else 0.0:.0f} units): {v.kind}"]
                      + v.details)
    rel_diff = np.abs(gk - yk) / np.maximum(np.abs(yk), torch.finfo(dt).tiny)
    out.margin = max(v.margin, float(rel_diff.max()) if yk.size else 0.0)
    return out


def _softcap_selection_near(y: np.ndarray, got_values: torch.Tensor, keep: np.ndarray, u: float, got_tok: int,
                            dt) -> bool:
    """A soft-capped row whose draw lies among values the soft-cap saturates
    (or nearly so): there the kernels' tanh and the CPU's may round a value
    to neighbouring representable numbers, which reorders near-equal values
    and moves the draw by whole elements.  Accepted when the kernel's
    filtered values are the oracle's ``y`` within ``SOFTCAP_ULPS`` units of
    the dtype on the kept elements (exactly -inf elsewhere) and the draw lies
    within the rounding doubt of ``got_tok``'s interval on the kernel's own
    values."""
    g = got_values.to(dt).double().numpy()
    if not np.array_equal(np.isfinite(g), keep):
        return False
    mant = {torch.float32: 23, torch.bfloat16: 7, torch.float16: 10}[dt]
    yk, gk = y[keep], g[keep]
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(yk), torch.finfo(dt).tiny))) - mant)
    if yk.size == 0 or float(np.max(np.abs(gk - yk) / ulp)) > SOFTCAP_ULPS[dt]:
        return False
    ok, _ = selection_near(torch.from_numpy(g).to(dt), u, got_tok)
    return ok


def greedy_near(filt: torch.Tensor, got_tok: int, expect: int) -> tuple:
    """(acceptable, relative gap) for a greedy pick: ``got_tok`` may replace
    the oracle's first maximal probability only if a relative perturbation of
    ``RK`` of the two float64 probabilities lets it win the first-index
    argmax of the dtype-rounded values."""
    dt = filt.dtype
    p64 = F.softmax(filt.double(), dim=-1).numpy()
    pg, pe = p64[got_tok], p64[expect]
    if pg <= 0.0:
        return False, float("inf")
    rg = float(_rn(np.array([pg * (1.0 + RK)]), dt)[0])
    re_ = float(_rn(np.array([pe * (1.0 - RK)]), dt)[0])
    wins = rg > re_ or (rg == re_ and got_tok < expect)
    return bool(wins), abs(pe - pg) / pe


def summarise(verdicts: List[RowVerdict]) -> dict:
    out = {k: 0 for k in ("EXACT", "TIE", "NEAR", "CONSEQ", "MISMATCH")}
    for v in verdicts:
        out[v.kind] += 1
    out["max_margin"] = max([v.margin for v in verdicts] + [0.0])
    return out


# --------------------------------------------------------------------------
# Speculative verify (speculative.py:54-84)
# --------------------------------------------------------------------------

def _ratio(pv: float, qv: float, dt) -> float:
    q1 = float(_rn(np.array([float(_rn(np.array([qv]), dt)[0]) + 1e-10]), dt)[0])
    return min(1.0, float(_rn(np.array([pv / q1]), dt)[0]))


def _accept_window(p64: float, q64: float, ratio_oracle: float, u: float, dt) -> tuple:
    rs = [_ratio(float(_rn(np.array([p64 * a]), dt)[0]), float(_rn(np.array([q64 * c]), dt)[0]), dt)
          for a in (1.0 - RK, 1.0, 1.0 + RK) for c in (1.0 - RK, 1.0, 1.0 + RK)]
    lo = min(rs + [ratio_oracle]) * (1.0 - RK)
    hi = max(rs + [ratio_oracle]) * (1.0 + RK)
    dist = 0.0 if lo <= u <= hi else min(abs(u - lo), abs(u - hi))
    return bool(lo <= u <= hi), dist


def _residual_doubt(pt: torch.Tensor, pd: torch.Tensor, p64: np.ndarray, q64: np.ndarray) -> tuple:
    """The oracle's residual weights (``speculative.py:73-74`` as the oracle
    evaluates them) normalised and cumulated in ascending index order, and the
    per-position doubt of a kernel that evaluates the same expression on
    correctly rounded probabilities (up to ``RK``)."""
    dt = pt.dtype
    r = torch.clamp(pt - pd, min=0)
    r = r / (r.sum() + 1e-10)
    w_or = r.double().numpy()
    use_p = float(w_or.sum()) <= 0.0
    if use_p:
        w_or = pt.double().numpy()
    pk, qk = _rn(p64, dt), _rn(q64, dt)
    ambp = np.abs(_rn(p64 * (1.0 + RK), dt) - _rn(p64 * (1.0 - RK), dt))
    ambq = np.abs(_rn(q64 * (1.0 + RK), dt) - _rn(q64 * (1.0 - RK), dt))
    if use_p:
        wk, amb = pk, ambp
    else:
        wk = np.maximum(_rn(pk - qk, dt), 0.0)
        amb = np.where((pk + ambp > qk - ambq), ambp + ambq, 0.0)
    so, sk = float(w_or.sum()), float(wk.sum())
    if sk <= 0.0:
        sk = so
    c_or = np.cumsum(w_or) / so
    c_k = np.cumsum(wk) / sk
    return c_or, np.abs(c_or - c_k) + np.cumsum(amb) / sk + 1e-12


def _interval_ok(c: np.ndarray, d: np.ndarray, j: int, t: float) -> tuple:
    lo, dlo = (c[j - 1], d[j - 1]) if j > 0 else (0.0, 0.0)
    hi, dhi = c[j], d[j]
    if hi <= lo:   # an empty interval: a zero weight is never drawn
        return False, float("inf")
    return bool(lo - dlo <= t < hi + dhi), max(0.0, lo - t, t - hi)


def _top_p_alternatives(row: torch.Tensor, p: O.RowParams, softcap: float = 0.0, cap_per_group: int = 16) -> list:
    """Filtered rows (dtype, [V]) whose kept sets differ from the oracle's
    only in the kept count of a top-p boundary value group, for every count
    the rounding doubt of the cumulative sums allows (``_top_p_count_range``):
    the group of the smallest kept value and the group of the largest value
    that top-p removed.  Members of a group are kept lowest index first, as
    the kernels keep them.  Empty when top-p is off or its cut is certain."""
    if p.top_p is None or not (0.0 < p.top_p < 1.0):
        return []
    dt = row.dtype
    y_t = O.pre_filter_values(row[None], p.temperature, 1.0, None, softcap)[0]
    y = y_t.double().numpy()
    stage = O._top_k(y_t[None].clone(), p.top_k or None)
    stage = O._min_p(stage, p.min_p or None)
    surv = ~np.isneginf(stage[0].double().numpy())
    _, filt = O.filtered_probs(row, p, softcap)
    keep = ~np.isneginf(filt.double().numpy())
    groups = []
    if keep.any():
        groups.append(float(y[keep].min()))
    if (surv & ~keep).any():
        groups.append(float(y[surv & ~keep].max()))
    alts = []
    for v in groups:
        grp = np.nonzero(y == v)[0]
        lo_n, hi_n, _ = _top_p_count_range(y, surv, grp, p.top_p, dt)
        cur = int(keep[grp].sum())
        for c in range(lo_n, min(hi_n, lo_n + cap_per_group) + 1):
            if c == cur:
                continue
            k2 = keep.copy()
            k2[grp] = False
            k2[grp[:c]] = True
            alts.append(torch.from_numpy(np.where(k2, y, -np.inf)).to(dt))
    return alts


def classify_spec(target: torch.Tensor, draft: torch.Tensor, draft_ids: torch.Tensor, p: O.RowParams,
                  u_accept: torch.Tensor, u_resample: torch.Tensor, got_n, got_tokens, softcap: float = 0.0,
                  ref: Optional[List[O.SpecResult]] = None):
    """Per sequence: EXACT, NEAR (the first difference is an accept decision
    whose ``u`` lies within the doubt of the ratio, or a resampled / bonus
    token whose cumulative interval lies within the doubt of the draw) or
    MISMATCH.  Where a row's top-p cut is itself open under rounding, the
    filtered rows with the other allowed kept counts (``_top_p_alternatives``)
    are tried too.  Returns (summary, [(kind, distance)], oracle results)."""
    if ref is None:
        ref = O.speculative_verify(target, draft, draft_ids, p, u_accept, u_resample, softcap=softcap)
    B, K = draft_ids.shape
    gn = [int(v) for v in got_n]
    gt = [[int(t) for t in row] for row in got_tokens]
    out = []
    for b in range(B):
        r = ref[b]
        n = gn[b]
        toks = gt[b][:n + 1]
        if n == r.n_accepted and toks == r.tokens:
            out.append(("EXACT", 0.0))
            continue
        m = min(n, r.n_accepted)
        if n != r.n_accepted or toks[:m] != r.tokens[:m]:
            if toks[:m] != r.tokens[:m]:
                out.append(("MISMATCH", float("inf")))
                continue
            pt, ft = O.filtered_probs(target[b, m], p, softcap)
            pd, fd = O.filtered_probs(draft[b, m], p, softcap)
            d = int(draft_ids[b, m])
            p64 = float(torch.softmax(ft.double(), -1)[d])
            q64 = float(torch.softmax(fd.double(), -1)[d])
            ok, dist = _accept_window(p64, q64, r.accept_ratio[m], float(u_accept[b, m]), pt.dtype)
            if not ok:
                for at in [ft] + _top_p_alternatives(target[b, m], p, softcap):
                    for ad in [fd] + _top_p_alternatives(draft[b, m], p, softcap):
                        if at is ft and ad is fd:
                            continue
                        pa = torch.softmax(at, -1)
                        qa = torch.softmax(ad, -1)
                        ra = _ratio(float(pa[d]), float(qa[d]), pt.dtype)
                        ok2, d2 = _accept_window(float(torch.softmax(at.double(), -1)[d]),
                                                 float(torch.softmax(ad.double(), -1)[d]), ra,
                                                 float(u_accept[b, m]), pt.dtype)
                        if ok2:
                            ok, dist = True, d2
                            break
                    if ok:
                        break
            out.append(("NEAR" if ok else "MISMATCH", dist))
            continue
        t = float(np.float64(np.float32(u_resample[b])))
        g = toks[-1]
        if n < K:   # residual at position n
            pt, ft = O.filtered_probs(target[b, n], p, softcap)
            pd, fd = O.filtered_probs(draft[b, n], p, softcap)
            p64 = torch.softmax(ft.double(), -1).numpy()
            q64 = torch.softmax(fd.double(), -1).numpy()
            c, dd = _residual_doubt(pt, pd, p64, q64)
            ok, dist = _interval_ok(c, dd, g, t) if 0 <= g < c.size else (False, float("inf"))
            if not ok:
                for at in [ft] + _top_p_alternatives(target[b, n], p, softcap):
                    for ad in [fd] + _top_p_alternatives(draft[b, n], p, softcap):
                        if at is ft and ad is fd:
                            continue
                        ca, da = _residual_doubt(torch.softmax(at, -1), torch.softmax(ad, -1),
                                                 torch.softmax(at.double(), -1).numpy(),
                                                 torch.softmax(ad.double(), -1).numpy())
                        if 0 <= g < ca.size and _interval_ok(ca, da, g, t)[0]:
                            ok, dist = True, 0.0
                            break
                    if ok:
                        break
        else:       # bonus from target position K
            _, ft = O.filtered_probs(target[b, K], p, softcap)
            ok, dist = selection_near(ft, float(u_resample[b]), g)
            if not ok:
                for at in _top_p_alternatives(target[b, K], p, softcap):
                    if selection_near(at, float(u_resample[b]), g)[0]:
                        ok, dist = True, 0.0
                        break
        out.append(("NEAR" if ok else "MISMATCH", dist))
    kinds = [k for k, _ in out]
    summ = {k: kinds.count(k) for k in ("EXACT", "NEAR", "MISMATCH")}
    return summ, out, ref

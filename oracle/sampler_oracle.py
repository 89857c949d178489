"""Op-for-op CPU restatement of the reference token sampler (test infrastructure).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may use this module, and only as the reference the kernels are compared
with / the timed CPU baseline.

The reference sampler is plain PyTorch; its arithmetic *is* the sequence of
ATen calls it makes.  This restatement therefore performs the same ATen calls,
in the same order and in the same dtype, so that it reproduces the reference's
rounding bit for bit (checked against vectors produced by the reference file
itself, ``tests/golden/``).  Where the reference leaves a choice open the
build's convention is stated and marked CONVENTION.

Stage order (reference ``sampling.py:26-51``; soft-cap is an extension):
    [soft-cap] -> repetition penalty -> temperature -> top-k -> min-p -> top-p
    -> softmax -> select -> stop / log-prob

Pinning of each function (what checks it besides retyping):
    filter_logits        golden vectors written by running the reference's
                         ``apply_sampling_filters`` (tests/golden), the 1x4
                         known-answer test of ``tests/unit/test_models.py:50-59``,
                         brute-force fp64 invariants (top-k keeps >= k and all
                         ties, top-p keeps the argmax and a mass >= top_p,
                         monotonicity in top_p).
    soft_cap             closed form tanh(x/c)*c checked against numpy fp64
                         within 2 ulp; tanh limits (x -> +-inf gives +-c).
    select_token         CONVENTION (inverse CDF).  Pinned by properties: a
                         uniform grid of u reproduces the probabilities as
                         selection frequencies, u -> 0 gives the top token,
                         one-hot rows, T<=0 equals torch.argmax.
    sample_rows          composition of the above, per-row loop of
                         ``engine.py:114-139``; stop membership checked on
                         hand-built cases.
    token_logprob        against the float64 log-softmax of the filtered row
                         (within the dtype's rounding of the kept mass and its
                         log, as torch evaluates log_softmax), -log n on rows
                         of n equal kept values, planted mistakes (the
                         unfiltered row, a missing shift) fail.
    speculative_verify   accept rule and residual of ``speculative.py:63-75``;
                         pinned by p == q (always accept), disjoint supports
                         (always reject, residual == p), and a chi-square test
                         that emitted tokens follow the target distribution.
    filtered_probs,      the parts of speculative_verify, pinned with it.
    residual_token
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np
import torch
import torch.nn.functional as F

NEG_INF = float("-inf")


# --------------------------------------------------------------------------
# Filter stages.  Each helper mutates / returns a [B, V] tensor in the input
# dtype exactly as the corresponding reference lines do.
# --------------------------------------------------------------------------

def soft_cap(x: torch.Tensor, cap: float) -> torch.Tensor:
    """Final-logit soft-cap ``tanh(x / cap) * cap`` (formula of the reference's
    attention soft-cap, ``models/attention/causal.py:109-110``).  Off if cap <= 0."""
    if cap is None or cap <= 0:
        return x
    return torch.tanh(x / cap) * cap


def _penalise_history(x: torch.Tensor, penalty: float, history: Optional[Sequence[int]]) -> torch.Tensor:
    """Repetition penalty, reference ``sampling.py:27-31``.

    Presence semantics: the ids are de-duplicated (``unique``), positives are
    divided by the penalty and non-positives multiplied, each in the tensor's
    dtype with the Python scalar as the second operand.  ``x`` is the clone,
    modified in place through advanced indexing."""
    if penalty == 1.0 or not history:
        return x
    ids = torch.tensor(list(history), device=x.device).unique()
    cols = x[:, ids]
    x[:, ids] = torch.where(cols > 0, cols / penalty, cols * penalty)
    return x


def _scale_temperature(x: torch.Tensor, temperature: float) -> torch.Tensor:
    """``sampling.py:33-34``: divide by T only when T > 0 (T == 0 means greedy)."""
    return x / temperature if temperature > 0 else x


def _top_k(x: torch.Tensor, k: Optional[int]) -> torch.Tensor:
    """``sampling.py:36-38``: remove everything strictly below the k-th largest
    value; all ties with the k-th value survive."""
    if k is None or k <= 0:
        return x
    kth = torch.topk(x, min(k, x.size(-1))).values[:, -1:]
    x[x < kth] = NEG_INF
    return x


def _min_p(x: torch.Tensor, min_p: Optional[float]) -> torch.Tensor:
    """``sampling.py:40-43``: remove tokens whose softmax probability is below
    ``min_p`` times the largest probability (both in the tensor's dtype)."""
    if min_p is None or min_p <= 0:
        return x
    probs = F.softmax(x, dim=-1)
    floor = min_p * probs.max(dim=-1, keepdim=True).values
    x[probs < floor] = NEG_INF
    return x


def _top_p(x: torch.Tensor, top_p: Optional[float], stable: bool) -> torch.Tensor:
    """``sampling.py:45-51``: nucleus filter on the descending sort.

    A sorted position is removed when its exclusive cumulative probability
    (inclusive cumsum minus its own probability, each rounded in the tensor's
    dtype) reaches ``top_p``.  The reference sorts with torch's default
    (unstable) sort; CONVENTION: the oracle sorts stably (``stable=True``) so
    that within a tie group the lower vocabulary indices come first.  Pass
    ``stable=False`` to reproduce the reference's own order."""
    if top_p is None or not (0 < top_p < 1.0):
        return x
    vals, order = torch.sort(x, descending=True, stable=stable)
    p_sorted = F.softmax(vals, dim=-1)
    exclusive = torch.cumsum(p_sorted, dim=-1) - p_sorted
    vals[exclusive >= top_p] = NEG_INF
    return vals.scatter(1, order, vals)


def filter_logits(
    logits: torch.Tensor,
    temperature: float = 1.0,
    top_k: Optional[int] = None,
    top_p: Optional[float] = None,
    min_p: Optional[float] = None,
    repetition_penalty: float = 1.0,
    past_tokens: Optional[Sequence[int]] = None,
    softcap: float = 0.0,
    stable: bool = True,
) -> torch.Tensor:
    """Restatement of ``apply_sampling_filters`` (``sampling.py:16-53``).

    Returns a new ``[B, V]`` tensor (input dtype) with removed entries set to
    ``-inf``; the input is not modified (reference clones at ``:26``)."""
    x = logits.clone()
    if softcap and softcap > 0:
        x = soft_cap(x, softcap)
    x = _penalise_history(x, repetition_penalty, past_tokens)
    x = _scale_temperature(x, temperature)
    x = _top_k(x, top_k)
    x = _min_p(x, min_p)
    x = _top_p(x, top_p, stable)
    return x


def pre_filter_values(logits: torch.Tensor, temperature: float = 1.0, repetition_penalty: float = 1.0,
                      past_tokens: Optional[Sequence[int]] = None, softcap: float = 0.0) -> torch.Tensor:
    """The values the filters compare: soft-cap, penalty and temperature only."""
    x = logits.clone()
    if softcap and softcap > 0:
        x = soft_cap(x, softcap)
    x = _penalise_history(x, repetition_penalty, past_tokens)
    return _scale_temperature(x, temperature)


# --------------------------------------------------------------------------
# Selection (CONVENTION) -- replaces torch.multinomial of sampling.py:61
# --------------------------------------------------------------------------

def selection_order(filtered_row: torch.Tensor) -> torch.Tensor:
    """Descending filtered value; ties by ascending vocabulary index."""
    return torch.sort(filtered_row, descending=True, stable=True).indices


def select_token(filtered_row: torch.Tensor, u: float, temperature: float) -> int:
    """Pick one token from a filtered ``[V]`` row.

    ``probs = softmax(filtered)`` in the row's dtype, as ``sampling.py:58``.
    ``T <= 0``: ``torch.argmax(probs)`` (first maximal index), as ``:59-60``.
    Otherwise CONVENTION: inverse CDF with the caller's uniform ``u`` in
    [0, 1).  Tokens are visited in ``selection_order``; their probabilities are
    accumulated in float64; the token is the first whose inclusive cumulative
    sum exceeds ``u * total``."""
    probs = F.softmax(filtered_row, dim=-1)
    if temperature <= 0:
        return int(torch.argmax(probs))
    order = selection_order(filtered_row)
    cum = torch.cumsum(probs[order].double(), dim=0)
    target = float(np.float64(np.float32(u)) * cum[-1].item())
    j = int(torch.searchsorted(cum, torch.tensor([target], dtype=torch.float64), right=True)[0])
    j = min(j, cum.numel() - 1)
    return int(order[j])


def token_logprob(filtered_row: torch.Tensor, token: int) -> float:
    """``F.log_softmax(filtered).gather(tok)`` of ``sampling.py:97-98`` (row dtype)."""
    return float(F.log_softmax(filtered_row, dim=-1)[token].float())


# --------------------------------------------------------------------------
# Batched, heterogeneous rows (engine.py:114-139 applies each request's own
# parameters to its own [1, V] slice)
# --------------------------------------------------------------------------

@dataclass
class RowParams:
    temperature: float = 1.0
    top_k: int = 0          # 0 == off
    top_p: float = 1.0      # 1.0 == off
    min_p: float = 0.0      # 0 == off
    repetition_penalty: float = 1.0
    history: List[int] = field(default_factory=list)
    stop_ids: List[int] = field(default_factory=list)


@dataclass
class RowResult:
    token: int
    finished: bool
    logprob: float
    filtered: torch.Tensor  # [V], input dtype


def sample_rows(logits: torch.Tensor, params: Sequence[RowParams], uniforms: Sequence[float],
                softcap: float = 0.0, finished_in: Optional[Sequence[bool]] = None,
                want_filtered: bool = True) -> List[RowResult]:
    """One ``[1, V]`` filter + select per row, the way ``engine.py:119-120`` does.

    Stop handling follows ``engine.py:123-127``: a row is finished when it was
    already finished or its token is in the row's stop set."""
    out: List[RowResult] = []
    for b, p in enumerate(params):
        row = logits[b:b + 1]
        filt = filter_logits(row, p.temperature, p.top_k or None, p.top_p, p.min_p or None,
                             p.repetition_penalty, p.history if p.repetition_penalty != 1.0 else None,
                             softcap=softcap)
        tok = select_token(filt[0], float(uniforms[b]), p.temperature)
        done = bool(finished_in[b]) if finished_in is not None else False
        done = done or (tok in set(int(s) for s in p.stop_ids))
        out.append(RowResult(tok, done, token_logprob(filt[0], tok), filt[0] if want_filtered else None))
    return out


# --------------------------------------------------------------------------
# Speculative decoding verify (speculative.py:30-87), batched over sequences
# --------------------------------------------------------------------------

@dataclass
class SpecResult:
    n_accepted: int
    tokens: List[int]         # accepted drafts, then the resampled / bonus token
    accept_ratio: List[float]


def filtered_probs(row: torch.Tensor, p: RowParams, softcap: float = 0.0) -> torch.Tensor:
    """Post-filter softmax of one [V] row (speculative.py:39-40, 58-59 with the
    full filter set of sampling.py in place of ``_topk_filter``)."""
    filt = filter_logits(row[None], p.temperature, p.top_k or None, p.top_p, p.min_p or None, softcap=softcap)
    return F.softmax(filt, dim=-1)[0], filt[0]


def residual_token(p: torch.Tensor, q: torch.Tensor, u: float) -> int:
    """Residual resample at the first rejection, ``speculative.py:73-75``:
    ``r = clamp(p - q, 0) / (sum + 1e-10)``.  CONVENTION: inverse CDF over ``r``
    in ascending vocabulary order, float64 accumulation; if ``r`` is all zero
    (p == q exactly) the target distribution ``p`` is used instead."""
    r = torch.clamp(p - q, min=0)
    r = r / (r.sum() + 1e-10)
    w = r.double()
    if float(w.sum()) <= 0.0:
        w = p.double()
    cum = torch.cumsum(w, dim=0)
    target = float(np.float64(np.float32(u)) * cum[-1].item())
    j = int(torch.searchsorted(cum, torch.tensor([target], dtype=torch.float64), right=True)[0])
    return min(j, cum.numel() - 1)


def speculative_verify(target: torch.Tensor, draft: torch.Tensor, draft_ids: torch.Tensor, p: RowParams,
                       u_accept: torch.Tensor, u_resample: torch.Tensor, softcap: float = 0.0) -> List[SpecResult]:
    """Accept / resample / bonus for ``B`` sequences of ``K`` drafts.

    target [B, K+1, V], draft [B, K, V], draft_ids [B, K], u_accept [B, K],
    u_resample [B].  Per position i (``speculative.py:54-77``):
    ``ratio = min(1, p[d] / (q[d] + 1e-10))``; accept iff ``u_accept < ratio``;
    at the first rejection sample the residual with ``u_resample``; if all K
    are accepted sample the bonus token from target position K
    (``speculative.py:79-84``) with ``u_resample`` and ``select_token``."""
    B, K = draft_ids.shape
    results: List[SpecResult] = []
    for b in range(B):
        toks: List[int] = []
        ratios: List[float] = []
        n_acc = 0
        rejected = False
        for i in range(K):
            pt, _ = filtered_probs(target[b, i], p, softcap)
            pd, _ = filtered_probs(draft[b, i], p, softcap)
            d = int(draft_ids[b, i])
            ratio = (pt[d:d + 1] / (pd[d:d + 1] + 1e-10)).clamp(max=1.0)
            ratios.append(float(ratio))
            if bool(u_accept[b, i:i + 1].float() < ratio):
                n_acc += 1
                toks.append(d)
            else:
                toks.append(residual_token(pt, pd, float(u_resample[b])))
                rejected = True
                break
        if not rejected:
            _, filt = filtered_probs(target[b, K], p, softcap)
            toks.append(select_token(filt, float(u_resample[b]), p.temperature))
        results.append(SpecResult(n_acc, toks, ratios))
    return results

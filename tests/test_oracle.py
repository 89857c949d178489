"""The oracle pinned against the reference: golden vectors written by the
reference's own ``apply_sampling_filters``, the reference's known-answer test,
and closed forms / invariants for what no vector covers (CPU only)."""

import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import sampler_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "sampler_golden.npz")


def _golden():
    d = np.load(GOLDEN)
    meta = json.loads(bytes(d["meta_json"]).decode())
    cases = {}
    for name in meta["cases"]:
        if f"{name}/logits_bf16" in d:
            x = torch.from_numpy(d[f"{name}/logits_bf16"]).view(torch.bfloat16)
            ref = torch.from_numpy(d[f"{name}/filtered_bf16"]).view(torch.bfloat16)
        else:
            x = torch.from_numpy(d[f"{name}/logits_f32"])
            ref = torch.from_numpy(d[f"{name}/filtered_f32"])
        cases[name] = (x, ref, d[f"{name}/hist"], d[f"{name}/params"])
    return meta, cases


META, CASES = _golden()


def _row_filter(x, hist, params, b, stable, top_p_fn=None):
    T, k, p, mp, rp, cap = params[b]
    past = [int(v) for v in hist[b] if v >= 0]
    return O.filter_logits(x[b:b + 1], float(T), int(k) or None, float(p), float(mp) or None, float(rp),
                           past if rp != 1.0 else None, softcap=float(cap), stable=stable)[0]


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    if a.dtype == torch.bfloat16:
        return torch.equal(a.view(torch.int16), b.view(torch.int16))
    return torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_golden_meta():
    assert META["source"].startswith("src/forgeline/models/generation/sampling.py")
    assert len(CASES) == 9


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_matches_reference_bit_for_bit(name):
    """With the reference's unstable sort the restatement reproduces every
    filtered value, -inf position and tie-group member of the reference."""
    x, ref, hist, params = CASES[name]
    for b in range(x.size(0)):
        got = _row_filter(x, hist, params, b, stable=False)
        assert _same(got, ref[b]), f"{name} row {b}"


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_stable_convention_keeps_same_group_counts(name):
    """The build's convention (ties by ascending index) keeps the same number
    of members of every value group as the reference."""
    x, ref, hist, params = CASES[name]
    for b in range(x.size(0)):
        got = _row_filter(x, hist, params, b, stable=True)
        pre = O.pre_filter_values(x[b:b + 1], float(params[b][0]), float(params[b][4]),
                                  [int(v) for v in hist[b] if v >= 0] if params[b][4] != 1.0 else None,
                                  softcap=float(params[b][5]))[0].float()
        gk, rk = ~torch.isneginf(got.float()), ~torch.isneginf(ref[b].float())
        for v in torch.unique(pre[gk ^ rk]).tolist():
            grp = pre == v
            assert int((gk & grp).sum()) == int((rk & grp).sum()), f"{name} row {b} group {v}"


def test_planted_top_p_mistake_is_caught():
    """An oracle whose top-p uses the inclusive instead of the exclusive
    cumulative mass fails the golden vectors (the check has teeth)."""
    orig = O._top_p

    def mutant(x, top_p, stable):
        if top_p is None or not (0 < top_p < 1.0):
            return x
        vals, order = torch.sort(x, descending=True, stable=stable)
        cum = torch.cumsum(F.softmax(vals, dim=-1), dim=-1)
        vals[cum >= top_p] = float("-inf")
        return vals.scatter(1, order, vals)

    O._top_p = mutant
    try:
        bad = 0
        for name in ("plumbing_f32_4x512", "hetero_bf16_12x4096", "softcap_zipf_f32_4x4096"):
            x, ref, hist, params = CASES[name]
            bad += sum(not _same(_row_filter(x, hist, params, b, stable=False), ref[b]) for b in range(x.size(0)))
        assert bad > 0
    finally:
        O._top_p = orig


def test_planted_penalty_sign_mistake_is_caught():
    """Multiplying positives by the penalty (instead of dividing) fails."""
    orig = O._penalise_history

    def mutant(x, penalty, history):
        if penalty == 1.0 or not history:
            return x
        ids = torch.tensor(list(history)).unique()
        cols = x[:, ids]
        x[:, ids] = torch.where(cols > 0, cols * penalty, cols / penalty)
        return x

    O._penalise_history = mutant
    try:
        x, ref, hist, params = CASES["uniform_f32_6x4096"]
        assert any(not _same(_row_filter(x, hist, params, b, stable=False), ref[b]) for b in range(x.size(0)))
    finally:
        O._penalise_history = orig


def test_reference_known_answers():
    """tests/unit/test_models.py:50-59 of the reference, on the oracle."""
    logits = torch.tensor([[1.0, 2.0, 3.0, 4.0]])
    top1 = O.filter_logits(logits, top_k=1)
    assert torch.isinf(top1[0, :3]).all() and top1[0, 3] == 4.0
    nucleus = O.filter_logits(logits, top_p=0.5)
    assert torch.isinf(nucleus[0, 0])
    minp = O.filter_logits(logits, min_p=0.5)
    assert torch.isinf(minp[0, 0])
    rep = O.filter_logits(logits, repetition_penalty=2.0, past_tokens=[3])
    assert rep[0, 3] == 2.0


# --------------------------------------------------------------------------
# Closed forms and invariants
# --------------------------------------------------------------------------

def _rows(seed, B=8, V=777, scale=2.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, V, generator=g) * scale).to(dtype)


@pytest.mark.parametrize("k", [1, 5, 50, 776, 777, 1000])
def test_top_k_keeps_k_largest_and_ties(k):
    x = _rows(1)
    x[:, 10:20] = x[:, 5:6]  # a tie group
    for b in range(x.size(0)):
        f = O.filter_logits(x[b:b + 1], top_k=k)[0]
        kept = ~torch.isneginf(f)
        kth = np.sort(x[b].numpy())[::-1][min(k, x.size(1)) - 1]
        assert torch.equal(kept, torch.from_numpy(x[b].numpy() >= kth))
        assert int(kept.sum()) >= min(k, x.size(1))


def test_top_p_invariants():
    x = _rows(2, B=6, V=600)
    for b in range(x.size(0)):
        prev = None
        for p in (0.1, 0.3, 0.5, 0.7, 0.9, 0.99):
            kept = ~torch.isneginf(O.filter_logits(x[b:b + 1], top_p=p)[0])
            probs = torch.softmax(x[b].double(), 0)
            assert bool(kept[int(torch.argmax(x[b]))])                      # keeps the top token
            assert float(probs[kept].sum()) >= p - 1e-6                     # kept mass reaches top_p
            # minimal: dropping the smallest kept token falls below top_p
            smallest = probs[kept].min()
            assert float(probs[kept].sum() - smallest) < p + 1e-6
            if prev is not None:
                assert bool((prev & ~kept).sum() == 0)                      # monotone in top_p
            prev = kept


@pytest.mark.parametrize("mp", [0.01, 0.1, 0.5, 1.0])
def test_min_p_matches_fp64_rule_up_to_rounding(mp):
    x = _rows(3, B=6, V=500, scale=3.0)
    for b in range(x.size(0)):
        kept = ~torch.isneginf(O.filter_logits(x[b:b + 1], min_p=mp)[0])
        e = torch.exp(x[b].double() - x[b].double().max())
        exact = e >= mp
        diff = kept ^ exact
        # disagreements only where e is within a few float32 ulp of min_p
        assert bool((torch.abs(e[diff] - mp) <= 8 * 2.0 ** -24 * mp).all())


def test_softcap_closed_form():
    x = torch.linspace(-200, 200, 4001)
    got = O.soft_cap(x, 30.0).double().numpy()
    want = np.tanh(x.double().numpy() / 30.0) * 30.0
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - want) <= 2 * ulp + 1e-30)
    assert float(O.soft_cap(torch.tensor([float("inf")]), 30.0)) == 30.0
    assert float(O.soft_cap(torch.tensor([float("-inf")]), 30.0)) == -30.0
    assert torch.equal(O.soft_cap(x, 0.0), x)


def test_temperature_is_ieee_division():
    x = _rows(4, B=1, V=1000)
    y = O.pre_filter_values(x, temperature=0.7)
    assert torch.equal(y, x / torch.tensor(0.7, dtype=torch.float32))
    assert torch.equal(O.pre_filter_values(x, temperature=0.0), x)


def test_penalty_presence_semantics():
    x = torch.tensor([[2.0, -2.0, 0.0, 4.0]])
    y = O.filter_logits(x, repetition_penalty=2.0, past_tokens=[0, 0, 1, 2])
    assert y[0].tolist() == [1.0, -4.0, 0.0, 4.0]   # duplicates penalise once; 0 stays 0


def test_select_token_properties():
    g = torch.Generator().manual_seed(5)
    row = torch.randn(50, generator=g)
    filt = O.filter_logits(row[None], top_p=0.9)[0]
    probs = torch.softmax(filt, -1).double()
    # u -> 0 takes the first token of the order (the largest value)
    assert O.select_token(filt, 0.0, 1.0) == int(torch.argmax(filt))
    # T <= 0 is argmax (first maximal index)
    tie = torch.tensor([1.0, 3.0, 3.0, 2.0])
    assert O.select_token(tie, 0.3, 0.0) == 1
    # one-hot row
    oh = torch.full((10,), float("-inf"))
    oh[7] = 0.0
    assert all(O.select_token(oh, u, 1.0) == 7 for u in (0.0, 0.5, 0.999))
    # a uniform grid of u reproduces the probabilities as frequencies
    n = 20000
    counts = torch.zeros(50, dtype=torch.float64)
    for i in range(n):
        counts[O.select_token(filt, (i + 0.5) / n, 1.0)] += 1
    assert float((counts / n - probs).abs().max()) <= 2.0 / n + 1e-6


def test_select_token_ties_ascending_index():
    row = torch.tensor([0.0, 1.0, 1.0, 1.0, 0.5])
    # three equal tokens (1, 2, 3) share the first ~70% of the mass in index order
    probs = torch.softmax(row.double(), 0)
    p1 = float(probs[1])
    assert O.select_token(row, 0.5 * p1, 1.0) == 1
    assert O.select_token(row, 1.5 * p1, 1.0) == 2
    assert O.select_token(row, 2.5 * p1, 1.0) == 3


def _logprob_fp64(row: torch.Tensor, tok: int) -> float:
    """log p(tok) of the filtered row from float64 sums, the way torch's CPU
    log_softmax evaluates it: ``y[tok] - m - log(S)`` with ``S`` the sum of
    ``exp(y - m)`` over the kept values; for 16-bit rows ``S`` and ``log(S)``
    are each rounded to the dtype before the subtraction (measured on torch's
    CPU kernels: 0 differences in 152050 bf16 and fp16 values, against ~7 %
    for the correctly rounded ``y - m - log(S)``), and the result is rounded
    to the dtype."""
    dt = row.dtype
    y = row.double()
    kept = y[~torch.isneginf(y)]
    m = float(kept.max())
    S = float(torch.exp(kept - m).sum())
    if dt == torch.float32:
        return float(y[tok]) - m - math.log(S)
    rn = lambda v: float(torch.tensor(v, dtype=torch.float64).float().to(dt).double())  # noqa: E731
    lse = rn(math.log(rn(S)))
    return rn(float(torch.tensor(float(y[tok]) - m - lse, dtype=torch.float64).float()))


def _ulp(v: float, dtype) -> float:
    a = torch.tensor([abs(v)], dtype=torch.float64).to(dtype)
    nxt = torch.nextafter(a.float(), torch.tensor([float("inf")])).to(dtype) if dtype == torch.float32 else None
    if dtype == torch.float32:
        return float(nxt.double() - a.double())
    bits = a.view(torch.int16).to(torch.int32) + 1
    return float(bits.to(torch.int16).view(dtype).double() - a.double())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_token_logprob_against_float64(dtype):
    """``log_softmax(filtered)[tok]`` (sampling.py:97-98) within one unit of the
    dtype (float32: 8 ulp) of the value computed from float64 sums, on rows
    with -inf entries (filtered tokens) and ties."""
    g = torch.Generator().manual_seed(21)
    for V in (7, 512, 32000):
        x = (torch.randn(4, V, generator=g) * 3.0)
        x[:, 1:4] = x[:, :1]                             # a tie group
        x = x.to(dtype)
        for b in range(4):
            filt = O.filter_logits(x[b:b + 1], temperature=0.9, top_k=max(2, V // 3), top_p=0.95)[0]
            kept = torch.nonzero(~torch.isneginf(filt.float())).flatten().tolist()
            for tok in kept[:: max(1, len(kept) // 25)] + [0]:
                if tok not in kept:
                    continue
                want = _logprob_fp64(filt, tok)
                got = O.token_logprob(filt, tok)
                tol = (8 if dtype == torch.float32 else 1) * _ulp(want, dtype) + 1e-7
                assert abs(got - want) <= tol, (V, b, tok, got, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [1, 2, 3, 7, 50, 1000])
def test_token_logprob_uniform_kept_set_is_minus_log_n(dtype, n):
    """A kept set of n equal values (everything else -inf): every kept token
    has log-probability -log n, rounded to the dtype."""
    row = torch.full((n + 37,), float("-inf"))
    idx = torch.randperm(n + 37, generator=torch.Generator().manual_seed(n))[:n]
    row[idx] = 1.75
    row = row.to(dtype)
    want = torch.tensor(-math.log(n), dtype=torch.float64).to(dtype).double().item()
    for tok in idx[:5].tolist():
        got = O.token_logprob(row, tok)
        assert abs(got - want) <= _ulp(want, dtype) * (4 if dtype == torch.float32 else 1), (got, want)


def test_token_logprob_planted_mistakes_fail_the_float64_check():
    """Plausible mistakes fail the float64 check above: normalising over the
    unfiltered row, dropping the log-sum-exp term, or gathering the next index."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, 300, generator=g) * 2.0
    filt = O.filter_logits(x, temperature=1.0, top_k=40)[0]
    kept = torch.nonzero(~torch.isneginf(filt)).flatten().tolist()
    tok = kept[5]
    want = _logprob_fp64(filt, tok)
    mutants = [
        float(F.log_softmax(x[0], -1)[tok]),                 # unfiltered normaliser
        float(filt[tok] - filt[~torch.isneginf(filt)].max()),  # no log-sum-exp
        float(F.log_softmax(filt, -1)[kept[6]]),              # the next kept index
    ]
    for m in mutants:
        assert abs(m - want) > 8 * _ulp(want, torch.float32) + 1e-7


def test_sample_rows_stop_and_finished():
    x = torch.tensor([[0.0, 10.0, 0.0], [10.0, 0.0, 0.0], [0.0, 0.0, 10.0]])
    params = [O.RowParams(temperature=0.0, stop_ids=[1]), O.RowParams(temperature=0.0, stop_ids=[2]),
              O.RowParams(temperature=0.0)]
    res = O.sample_rows(x, params, [0.5, 0.5, 0.5], finished_in=[False, False, True])
    assert [r.token for r in res] == [1, 0, 2]
    assert [r.finished for r in res] == [True, False, True]


# --------------------------------------------------------------------------
# Speculative verify (speculative.py:54-84)
# --------------------------------------------------------------------------

def _spec_inputs(seed, B=3, K=4, V=64, rho=0.8):
    g = torch.Generator().manual_seed(seed)
    z1 = torch.randn(B, K + 1, V, generator=g)
    z2 = torch.randn(B, K, V, generator=g)
    return 2 * z1, 2 * (rho * z1[:, :K] + math.sqrt(1 - rho * rho) * z2), g


def test_spec_identical_distributions_always_accept():
    t, _, g = _spec_inputs(0)
    d = t[:, :-1].clone()
    ids = torch.randint(0, 64, (3, 4), generator=g)
    p = O.RowParams(temperature=1.0)
    res = O.speculative_verify(t, d, ids, p, torch.rand(3, 4, generator=g), torch.rand(3, generator=g))
    # ratio p/(p + 1e-10) rounds to 1 in float32 wherever p > ~1e-3; accept needs u < ratio
    for r in res:
        assert all(abs(x - 1.0) < 1e-6 or x > 0.99 for x in r.accept_ratio)


def test_spec_disjoint_support_residual_is_target():
    V = 32
    t = torch.full((1, 2, V), -1e9)
    t[..., :16] = torch.randn(1, 2, 16)
    d = torch.full((1, 1, V), -1e9)
    d[..., 16:] = torch.randn(1, 1, 16)
    p = O.RowParams(temperature=1.0)
    for u in (0.1, 0.4, 0.7, 0.95):
        res = O.speculative_verify(t, d, torch.tensor([[20]]), p, torch.tensor([[0.5]]), torch.tensor([u]))[0]
        assert res.n_accepted == 0
        pt, _ = O.filtered_probs(t[0, 0], p)
        assert res.tokens[0] == O.residual_token(pt, torch.zeros(V), u) and res.tokens[0] < 16


def test_spec_emits_target_distribution():
    """Chi-square: the first emitted token of speculative verify follows the
    target distribution whatever the draft (the method's defining property)."""
    V = 8
    g = torch.Generator().manual_seed(11)
    tl = torch.randn(V, generator=g)
    dl = torch.randn(V, generator=g)
    p = O.RowParams(temperature=1.0)
    pt = torch.softmax(tl.double(), 0)
    pd = torch.softmax(dl.double(), 0)
    n = 6000
    counts = np.zeros(V)
    t = tl.view(1, 1, V).expand(1, 2, V).contiguous()
    d = dl.view(1, 1, V)
    draws = torch.multinomial(pd.float(), n, replacement=True, generator=g)
    ua = torch.rand(n, generator=g)
    ur = torch.rand(n, generator=g)
    for i in range(n):
        r = O.speculative_verify(t, d, draws[i].view(1, 1), p, ua[i].view(1, 1), ur[i].view(1))[0]
        counts[r.tokens[0]] += 1
    expected = pt.numpy() * n
    chi2 = float(((counts - expected) ** 2 / expected).sum())
    assert chi2 < 24.3   # chi-square(7 dof) 0.999 quantile


# ---------------------------------------------------------------------------
# Full-distribution statistics (oracle/logprob_oracle.py)
# ---------------------------------------------------------------------------

def test_rowstats_oracle_uniform_rows():
    """Uniform logits: entropy log V, every label log-prob -log V, KL to itself
    0, log-sum-exp c + log V."""
    import math

    from oracle import logprob_oracle as L
    V = 1000
    x = torch.full((2, 3, V), 4.25)
    lab = torch.tensor([[0, 5, 999], [17, 2, 500]])
    assert torch.allclose(L.entropy_from_logits(x), torch.full((2, 3), math.log(V)), atol=1e-5)
    assert torch.allclose(L.token_logprobs_from_logits(x, lab), torch.full((2, 3), -math.log(V)), atol=1e-5)
    assert torch.allclose(L.kl_full_distribution(x, x), torch.zeros(2, 3), atol=1e-6)
    assert torch.allclose(L.logsumexp(x), torch.full((2, 3), 4.25 + math.log(V)), atol=1e-5)


def test_rowstats_oracle_two_point_closed_form():
    """V = 2: p = sigmoid(a - b); entropy -p ln p - q ln q; KL(p || r) by hand."""
    import math

    from oracle import logprob_oracle as L
    a, b, c, d = 1.3, -0.4, 0.2, 0.9
    p = 1.0 / (1.0 + math.exp(-(a - b)))
    r = 1.0 / (1.0 + math.exp(-(c - d)))
    H = -p * math.log(p) - (1 - p) * math.log(1 - p)
    KL = p * math.log(p / r) + (1 - p) * math.log((1 - p) / (1 - r))
    x = torch.tensor([[a, b]])
    y = torch.tensor([[c, d]])
    assert abs(float(L.entropy_from_logits(x)[0]) - H) < 1e-6
    assert abs(float(L.kl_full_distribution(x, y)[0]) - KL) < 1e-6
    assert abs(float(L.token_logprobs_from_logits(x, torch.tensor([1]))[0]) - math.log(1 - p)) < 1e-6


def test_rowstats_oracle_float64_brute_force_and_shift():
    """Random rows against explicit float64 formulas; adding a constant to a
    row changes none of the statistics."""
    from oracle import logprob_oracle as L
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4, 777, generator=g) * 3.0
    y = torch.randn(4, 777, generator=g) * 2.0
    lab = torch.randint(0, 777, (4,), generator=g)
    xd, yd = x.double(), y.double()
    lpx = xd - torch.logsumexp(xd, -1, keepdim=True)
    lpy = yd - torch.logsumexp(yd, -1, keepdim=True)
    H = -(lpx.exp() * lpx).sum(-1)
    KL = (lpx.exp() * (lpx - lpy)).sum(-1)
    LP = lpx.gather(1, lab[:, None])[:, 0]
    assert torch.allclose(L.entropy_from_logits(x).double(), H, atol=2e-5)
    assert torch.allclose(L.kl_full_distribution(x, y).double(), KL, atol=2e-5)
    assert torch.allclose(L.token_logprobs_from_logits(x, lab).double(), LP, atol=2e-5)
    assert torch.allclose(L.entropy_from_logits(x + 11.0), L.entropy_from_logits(x), atol=2e-5)
    assert torch.allclose(L.kl_full_distribution(x - 3.0, y + 5.0), L.kl_full_distribution(x, y), atol=2e-5)


def test_rowstats_oracle_ignore_index_and_neg_inf():
    """cross_entropy's ignore_index -100 gives log-prob -0.0; a -inf logit
    makes the reference's entropy NaN (0 * -inf) but leaves log-probs finite."""
    from oracle import logprob_oracle as L
    x = torch.tensor([[0.5, -1.0, 2.0, float("-inf")]])
    lp = L.token_logprobs_from_logits(x, torch.tensor([-100]))
    assert float(lp[0]) == 0.0 and str(float(lp[0])) == "-0.0"
    assert torch.isnan(L.entropy_from_logits(x)).all()
    assert torch.isfinite(L.token_logprobs_from_logits(x, torch.tensor([2]))).all()


def test_scalar_products_of_16_bit_tensors_use_float32_scalars():
    """``min_p * probs.max()`` (sampling.py:42) on a 16-bit tensor multiplies
    by the Python scalar in float32 and rounds the product once, whereas a
    comparison with a scalar (``>= top_p``) takes the scalar in the tensor's
    dtype; the kernels follow both."""
    g = torch.Generator().manual_seed(0)
    for dt in (torch.bfloat16, torch.float16):
        x = (torch.rand(4096, generator=g) * 2).to(dt)
        for s in (0.05, 0.1, 0.3):
            as_f32 = (torch.tensor(s, dtype=torch.float32) * x.float()).to(dt)
            as_dt = (torch.tensor(s).to(dt).float() * x.float()).to(dt)
            assert torch.equal(s * x, as_f32)
            assert not torch.equal(as_f32, as_dt)   # the two readings do differ
    b = torch.tensor([0.94921875, 0.953125], dtype=torch.bfloat16)
    assert (b >= 0.95).tolist() == [True, True]     # 0.95 compares as bf16 0.94921875


def test_greedy_compares_float32_probabilities():
    """T <= 0 is torch.argmax of the float32 probabilities: logits one ulp
    apart near zero have equal probabilities and the first index wins."""
    a = np.float32(0.1)
    row = torch.tensor([a, np.nextafter(a, np.float32(1.0)), -3.0], dtype=torch.float32)
    assert O.select_token(row, 0.5, 0.0) == 0
    assert int(torch.argmax(row)) == 1

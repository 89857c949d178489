"""lm_head with the sampler in its epilogue (``fl_lm_head_sample``, MI355X).

* The GEMM: the logits the kernel computes (its optional logits output) are
  the float64 product of the bf16 operands rounded to bf16, within one bf16
  unit where the fp32 accumulation lands next to a rounding boundary.
* The fused sampling: on the GEMM's own logits, the tokens and
  log-probabilities equal ``fl_sample``'s bit for bit (same rules, same
  arithmetic), and the oracle (the reference's filters and the
  inverse-CDF convention) classifies every row EXACT or NEAR.
* Rows the fused path leaves at FL_ROW_LIMIT (top-k off or above 64, more
  than 4096 values tied above the threshold) are sampled by ``fl_sample``
  through ``lm_head_sample``.
* Seeded random cases (batch 1 to 70, dim 64 to 4096, vocabularies of 100 to
  128256, soft-caps, per-row parameters and ragged history lengths): tokens
  and log-probabilities bit-equal to ``fl_sample`` on the GEMM's logits."""

import random

import pytest
import torch

from rl_project_amd import _lib, sample_tokens, workloads
from rl_project_amd.lmhead import LmHeadPlan, lm_head_sample
from tests.helpers import classify_workload

pytestmark = pytest.mark.gpu


def _operands(B, D, V, seed, scale=2.5):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(B, D, generator=g).to(torch.bfloat16)
    w = (torch.randn(V, D, generator=g) * (scale / D ** 0.5)).to(torch.bfloat16)
    return h.cuda(), w.cuda()


def _params(B, V, seed, top_k=None):
    g = torch.Generator().manual_seed(seed + 1)
    T = torch.rand(B, generator=g) * 1.4 + 0.1
    T[::7] = 0.0                                            # greedy rows
    K = torch.tensor([1, 5, 20, 50, 64, 33, 2, 40], dtype=torch.int32).repeat(B)[:B] if top_k is None \
        else torch.full((B,), top_k, dtype=torch.int32)
    P = torch.where(torch.rand(B, generator=g) < 0.6, torch.rand(B, generator=g) * 0.5 + 0.5, torch.ones(B))
    MP = torch.where(torch.rand(B, generator=g) < 0.3, torch.full((B,), 0.05), torch.zeros(B))
    RP = torch.where(torch.rand(B, generator=g) < 0.5, torch.rand(B, generator=g) * 0.3 + 1.0, torch.ones(B))
    hist = torch.randint(0, V, (B, 96), generator=g, dtype=torch.int32)
    U = torch.rand(B, generator=g)
    return dict(temperature=T, top_k=K, top_p=P, min_p=MP, repetition_penalty=RP, history=hist, uniforms=U)


def _check_logits(h, w, got):
    """|got - exact| <= one bf16 unit of the exact value (the final rounding,
    plus the accumulation landing across a rounding boundary) + the fp32
    accumulation bound D * 2^-24 * sum |h_d w_d| (the cancelling sums near
    zero); most logits equal the exact product rounded once."""
    ref = (h.double() @ w.double().T)
    mag = (h.double().abs() @ w.double().abs().T)
    rn = ref.to(torch.bfloat16)
    got = got.double()
    ulp = (rn.double().abs() * 2.0 ** -7).clamp_min(2.0 ** -133)
    tol = ulp + h.size(1) * 2.0 ** -24 * mag
    exact = (got == rn.double()).float().mean().item()
    worst = ((got - ref).abs() / tol).max().item()
    print(f"   logits: {exact * 100:.3f} % equal to the rounded float64 product; worst error {worst:.3f} of the bound",
          flush=True)
    assert worst <= 1.0 and exact > 0.99


@pytest.mark.parametrize("B,D,V,softcap", [(5, 256, 4099, 0.0), (24, 1024, 32000, 30.0), (64, 4096, 128256, 0.0)])
def test_fused_lm_head_matches_gemm_and_fl_sample(B, D, V, softcap):
    print(f"[lm_head fused] B={B} D={D} V={V} softcap={softcap}", flush=True)
    h, w = _operands(B, D, V, seed=B + V)
    kw = _params(B, V, seed=B)
    kd = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    plan = LmHeadPlan(h, w, softcap=softcap, return_logprobs=True, return_logits=True, **kd)
    plan.launch()
    torch.cuda.synchronize()
    out = plan.output
    assert out.status.tolist() == [0] * B, out.status.tolist()
    _check_logits(h, w, out.logits)
    # fl_sample over the GEMM's logits: the same tokens and log-probabilities, bit for bit
    ref = sample_tokens(out.logits, softcap=softcap, return_logprobs=True, **kd)
    torch.cuda.synchronize()
    assert torch.equal(ref.tokens, out.tokens), (ref.tokens.tolist(), out.tokens.tolist())
    assert torch.equal(ref.logprobs.view(torch.int32), out.logprobs.view(torch.int32))
    # the oracle on the GEMM's logits
    wl = workloads.SampleWorkload("lmhead", out.logits.cpu(), kw["temperature"], kw["top_k"], kw["top_p"], kw["min_p"],
                                  kw["repetition_penalty"], kw["history"], None, kw["uniforms"], softcap=softcap)
    summ, verdicts = classify_workload(wl, out.tokens)
    print(f"   oracle: {summ}", flush=True)
    assert summ["MISMATCH"] == 0, [(b, v.details) for b, v in enumerate(verdicts) if not v.ok][:4]
    # and without the logits output: the same tokens
    plan2 = LmHeadPlan(h, w, softcap=softcap, **kd)
    plan2.launch()
    torch.cuda.synchronize()
    assert torch.equal(plan2.tokens, out.tokens)


def test_rows_the_fused_path_cannot_decide():
    """top_k 0 and 65 (outside 1..64) and a row whose values tie above the
    threshold more than 4096 times report FL_ROW_LIMIT from the fused path;
    lm_head_sample samples them with fl_sample over the GEMM's logits."""
    B, D, V = 6, 512, 20000
    print(f"[lm_head limits] B={B} D={D} V={V}", flush=True)
    h, w = _operands(B, D, V, seed=7)
    # row 3: hidden state orthogonal to 6000 identical weight rows, which then
    # all give the same (largest) logit
    w[:6000] = 0
    w[:6000, 0] = 4.0
    h[:, 0] = 0
    h[3] = 0
    h[3, 0] = 1.0
    kw = dict(temperature=torch.full((B,), 0.9), top_k=torch.tensor([0, 65, 20, 10, 50, 1], dtype=torch.int32),
              top_p=torch.full((B,), 0.9), uniforms=torch.rand(B, generator=torch.Generator().manual_seed(3)))
    kd = {k: v.cuda() for k, v in kw.items()}
    plan = LmHeadPlan(h, w, return_logits=True, **kd)
    plan.launch()
    torch.cuda.synchronize()
    L = _lib.FL_ROW_LIMIT
    assert plan.status.tolist() == [L, L, 0, L, 0, 0], plan.status.tolist()
    out = lm_head_sample(h, w, return_logprobs=True, fused=True, **kd)
    ref = sample_tokens(plan.logits, return_logprobs=True, **kd)
    torch.cuda.synchronize()
    assert out.status.tolist() == [0] * B
    assert torch.equal(out.tokens, ref.tokens) and torch.equal(out.logprobs, ref.logprobs)
    assert int(out.tokens[3]) < 6000


def test_penalties_temperatures_and_overflow():
    """The fused path compares raw logits against per-row thresholds that the
    soft-cap, penalty and temperature map back from the bound; rows with a
    penalty below 1 (raising negative and lowering positive values the other
    way), tiny and zero temperatures, and a logit that overflows to +inf give
    fl_sample's tokens, log-probabilities and status bits.  A penalty that is
    not a positive finite number (rows 4 and 5) reports FL_ROW_LIMIT from the
    fused path; lm_head_sample then uses fl_sample."""
    B, D, V = 8, 256, 5000
    print(f"[lm_head edges] B={B} D={D} V={V}", flush=True)
    h, w = _operands(B, D, V, seed=21)
    h[2] = 0
    h[2, 0] = 2.0 ** 100
    w[7, 0] = 2.0 ** 100          # row 2: logit 7 overflows to +inf, the others are about 2^96
    g = torch.Generator().manual_seed(22)
    kw = dict(temperature=torch.tensor([0.8, 0.01, 0.0, 1.3, 0.8, 0.8, 0.05, 2.0]),
              top_k=torch.tensor([5, 20, 64, 1, 10, 10, 50, 33], dtype=torch.int32),
              top_p=torch.tensor([0.9, 1.0, 0.7, 1.0, 0.9, 0.9, 0.95, 0.8]),
              repetition_penalty=torch.tensor([0.7, 1.2, 0.5, 1.0, 0.0, -1.0, 1.5, 0.9]),
              history=torch.randint(0, V, (B, 64), generator=g, dtype=torch.int32),
              uniforms=torch.rand(B, generator=g))
    kd = {k: v.cuda() for k, v in kw.items()}
    plan = LmHeadPlan(h, w, return_logprobs=True, return_logits=True, **kd)
    plan.launch()
    torch.cuda.synchronize()
    ref = sample_tokens(plan.logits, return_logprobs=True, check_status=False, **kd)
    torch.cuda.synchronize()
    st, rst = plan.status.tolist(), ref.status.tolist()
    print(f"   fused status {st}, fl_sample status {rst}", flush=True)
    L = _lib.FL_ROW_LIMIT
    assert st[4] == L and st[5] == L
    assert rst[2] & _lib.FL_ROW_INF and st[2] == rst[2]
    for b in (0, 1, 3, 6, 7):
        assert st[b] == rst[b] == 0, (b, st[b], rst[b])
        assert int(plan.tokens[b]) == int(ref.tokens[b]), b
        assert plan.logprob[b].view(torch.int32).item() == ref.logprobs[b].view(torch.int32).item(), b
    out = lm_head_sample(h, w, return_logprobs=True, check_status=False, fused=True, **kd)
    torch.cuda.synchronize()
    assert out.status.tolist()[:2] + out.status.tolist()[3:] == rst[:2] + rst[3:]
    assert torch.equal(out.tokens[[0, 1, 3, 4, 5, 6, 7]], ref.tokens[[0, 1, 3, 4, 5, 6, 7]])


def test_batches_above_64_rows_run_in_groups():
    B, D, V = 100, 256, 8192
    print(f"[lm_head groups] B={B}", flush=True)
    h, w = _operands(B, D, V, seed=11)
    kw = _params(B, V, seed=12)
    kd = {k: v.cuda() for k, v in kw.items()}
    out = lm_head_sample(h, w, return_logits=True, fused=True, **kd)
    ref = sample_tokens(out.logits, **kd)
    torch.cuda.synchronize()
    assert torch.equal(out.tokens, ref.tokens)
    _check_logits(h, w, out.logits)


@pytest.mark.parametrize("first", [0, 12])
def test_random_lm_head_cases(first):
    for seed in range(first, first + 12):
        rng = random.Random(1000 + seed)
        B = rng.choice([1, 3, 16, 17, 40, 64, 70])
        D = rng.choice([64, 256, 1024, 4096])
        V = rng.choice([100, 4099, 32000, 50257, 128256])
        cap = rng.choice([0.0, 0.0, 30.0, 5.0])
        print(f"[lm_head random] seed={1000 + seed} B={B} D={D} V={V} softcap={cap}", flush=True)
        h, w = _operands(B, D, V, seed=1000 + seed, scale=rng.choice([1.0, 2.5, 8.0]))
        g = torch.Generator().manual_seed(2000 + seed)
        kw = dict(temperature=torch.tensor([rng.choice([0.0, 0.3, 0.8, 1.0, 1.5]) for _ in range(B)]),
                  top_k=torch.tensor([rng.choice([1, 2, 10, 50, 64]) for _ in range(B)], dtype=torch.int32),
                  top_p=torch.tensor([rng.choice([1.0, 0.5, 0.9, 0.99]) for _ in range(B)]),
                  min_p=torch.tensor([rng.choice([0.0, 0.0, 0.05, 0.3]) for _ in range(B)]),
                  repetition_penalty=torch.tensor([rng.choice([1.0, 1.3, 0.8]) for _ in range(B)]),
                  history=torch.randint(0, V, (B, rng.choice([1, 32, 300])), generator=g, dtype=torch.int32),
                  uniforms=torch.rand(B, generator=g))
        kd = {k: v.cuda() for k, v in kw.items()}
        out = lm_head_sample(h, w, softcap=cap, return_logprobs=True, return_logits=True, fused=True, **kd)
        ref = sample_tokens(out.logits, softcap=cap, return_logprobs=True, **kd)
        torch.cuda.synchronize()
        assert out.status.tolist() == [0] * B
        assert torch.equal(out.tokens, ref.tokens), seed
        assert torch.equal(out.logprobs.view(torch.int32), ref.logprobs.view(torch.int32)), seed


def test_argument_errors():
    h, w = _operands(4, 256, 1000, seed=1)
    with pytest.raises(NotImplementedError):
        LmHeadPlan(h.float(), w.float())
    with pytest.raises(ValueError):
        LmHeadPlan(h[:, :128], w)
    with pytest.raises(ValueError):   # dim not a multiple of 64
        LmHeadPlan(h[:, :100].contiguous(), w[:, :100].contiguous()).launch()


def test_last_position_view_of_prefill_states():
    """The reference takes the last position of the [B, T, D] hidden states
    (model.py:190,201): a strided view whose rows lie T*D apart.  Where the
    rows span more than the kernels' 32-bit offsets reach, the plan copies the
    view; tokens and log-probs equal those of the contiguous copy."""
    B, T, D, V = 17, 8192, 4096, 4099
    assert B * T * D > (1 << 29)
    g = torch.Generator(device="cuda").manual_seed(11)
    states = torch.empty(B, T, D, dtype=torch.bfloat16, device="cuda")
    states[:, -1, :] = torch.randn(B, D, generator=g, device="cuda").to(torch.bfloat16)
    W = (torch.randn(V, D, generator=g, device="cuda") * (2.5 / D ** 0.5)).to(torch.bfloat16)
    u = torch.rand(B, generator=g, device="cuda")
    kw = dict(temperature=0.8, top_k=20, top_p=0.9, uniforms=u, return_logprobs=True)
    view = states[:, -1, :]
    assert view.stride(0) == T * D
    a = lm_head_sample(view, W, fused=True, **kw)
    b = lm_head_sample(view.contiguous(), W, fused=True, **kw)
    torch.cuda.synchronize()
    assert a.tokens.tolist() == b.tokens.tolist()
    assert torch.equal(a.logprobs, b.logprobs)
    del states


def test_default_path_is_linear_then_fl_sample():
    """lm_head_sample without ``fused`` takes the path measured faster on
    MI355X at every batch size: torch's linear (the reference's lm_head) and
    then fl_sample, exactly -- and the fused kernels' logits stay within the
    bf16 rounding of the same products."""
    B, D, V = 24, 1024, 32000
    print(f"[lm_head default] B={B} D={D} V={V}", flush=True)
    h, w = _operands(B, D, V, seed=31)
    kw = _params(B, V, seed=32)
    kd = {k: v.cuda() for k, v in kw.items()}
    out = lm_head_sample(h, w, return_logprobs=True, return_logits=True, **kd)
    logits = torch.nn.functional.linear(h, w)
    ref = sample_tokens(logits, return_logprobs=True, **kd)
    fz = lm_head_sample(h, w, return_logits=True, fused=True, **kd)
    torch.cuda.synchronize()
    assert torch.equal(out.logits, logits)
    assert torch.equal(out.tokens, ref.tokens)
    assert torch.equal(out.logprobs.view(torch.int32), ref.logprobs.view(torch.int32))
    _check_logits(h, w, fz.logits)
    assert float((fz.logits.float() - logits.float()).abs().max()) <= \
        float(logits.float().abs().max()) * 2.0 ** -7

"""Parity of the fused full-distribution statistics kernel (token log-prob,
entropy, KL, log-sum-exp) with the oracle's restatement of the reference
functions (MI355X)."""

import pytest
import torch

from oracle import logprob_oracle as L
from rl_project_amd import entropy_from_logits, kl_full_distribution, row_stats, token_logprobs_from_logits

pytestmark = pytest.mark.gpu


def _close(got, ref, atol, rtol=1e-5):
    got, ref = got.cpu().double(), ref.double()
    both_nan = torch.isnan(got) & torch.isnan(ref)
    # (equal infinities: a label on a -inf logit has log-probability -inf)
    ok = both_nan | (got == ref) | ((got - ref).abs() <= atol + rtol * ref.abs())
    return bool(ok.all()), float(((got - ref).abs()[~ok]).max()) if bool((~ok).any()) else 0.0


@pytest.mark.parametrize("dtype,shape,scale", [
    (torch.float32, (2, 5, 32000), 3.0),
    (torch.bfloat16, (3, 7, 128256), 2.5),
    (torch.float16, (2, 3, 50257), 4.0),
    (torch.float32, (1, 1, 7), 1.0),          # one tiny row, V not a multiple of the chunk
    (torch.bfloat16, (4, 9, 4099), 8.0),      # sharp distributions
])
def test_row_stats_match_oracle(dtype, shape, scale):
    print(f"[row stats] {dtype} {shape} scale {scale}", flush=True)
    g = torch.Generator().manual_seed(sum(shape))
    x = (scale * torch.randn(*shape, generator=g)).to(dtype)
    y = (x.float() + 0.7 * torch.randn(*shape, generator=g)).to(dtype)
    lab = torch.randint(0, shape[-1], shape[:-1], generator=g)
    lab.view(-1)[::5] = -100  # ignored targets
    st = row_stats(x.cuda(), lab.cuda(), y.cuda(), entropy=True, lse=True)
    torch.cuda.synchronize()
    ok, err = _close(st.logprob, L.token_logprobs_from_logits(x, lab), 2e-5)
    assert ok, ("logprob", err)
    ign = (lab == -100)
    assert bool((st.logprob.cpu()[ign] == 0).all()) and bool(torch.signbit(st.logprob.cpu()[ign]).all())
    ok, err = _close(st.entropy, L.entropy_from_logits(x), 2e-5)
    assert ok, ("entropy", err)
    ok, err = _close(st.kl, L.kl_full_distribution(x, y), 2e-5)
    assert ok, ("kl", err)
    ok, err = _close(st.lse, L.logsumexp(x), 2e-5, 1e-6)
    assert ok, ("lse", err)


def test_reference_signatures_and_strided_rows():
    """The three drop-ins on a [B, T, V] slice with a row stride above V."""
    B, T, V = 2, 6, 30011
    g = torch.Generator().manual_seed(4)
    base = torch.randn(B, T, V + 13, generator=g) * 2.0
    x = base[..., :V]                      # rows V + 13 apart
    y = (torch.randn(B, T, V + 13, generator=g) * 2.0)[..., 5:5 + V]
    lab = torch.randint(0, V, (B, T), generator=g)
    xd, yd = base.cuda()[..., :V], y.cuda()
    lp = token_logprobs_from_logits(xd, lab.cuda())
    h = entropy_from_logits(xd)
    kl = kl_full_distribution(xd, yd)
    assert lp.shape == (B, T) and h.shape == (B, T) and kl.shape == (B, T) and lp.dtype == torch.float32
    assert _close(lp, L.token_logprobs_from_logits(x, lab), 2e-5)[0]
    assert _close(h, L.entropy_from_logits(x), 2e-5)[0]
    assert _close(kl, L.kl_full_distribution(x, y), 2e-5)[0]
    assert _close(kl_full_distribution(xd, xd), torch.zeros(B, T), 1e-6)[0]


def test_neg_inf_and_bad_labels():
    """-inf logits: entropy NaN as the reference's 0 * -inf, log-probs finite;
    an out-of-range label raises as cross_entropy does."""
    x = torch.randn(4, 1000)
    x[0, 10] = float("-inf")
    x[1, :500] = float("-inf")   # whole chunks of -inf before the first finite value
    x[3, :] = float("-inf")      # every logit -inf: NaN throughout, as log_softmax gives
    lab = torch.tensor([3, 700, 999, 5])
    st = row_stats(x.cuda(), lab.cuda(), entropy=True)
    ref_h = L.entropy_from_logits(x)
    assert _close(st.entropy, ref_h, 2e-5)[0]
    assert _close(st.logprob, L.token_logprobs_from_logits(x, lab), 2e-5)[0]
    with pytest.raises(IndexError):
        token_logprobs_from_logits(x.cuda(), torch.tensor([3, 1000, 1, 2]).cuda())


def test_random_row_stats_cases():
    """Seeded random shapes, dtypes and value ranges, with -inf entries and
    ignored targets: every statistic within the tolerances above."""
    import random
    for seed in range(40):
        rng = random.Random(seed)
        dt = rng.choice([torch.float32, torch.bfloat16, torch.float16])
        R = rng.choice([1, 7, 33])
        V = rng.choice([2, 100, 4099, 50257, 151936])
        scale = rng.choice([0.1, 1.0, 5.0, 20.0])
        g = torch.Generator().manual_seed(seed)
        x = scale * torch.randn(R, V, generator=g)
        y = x + rng.choice([0.0, 0.1, 2.0]) * torch.randn(R, V, generator=g)
        if rng.random() < 0.3:
            x[torch.rand(R, V, generator=g) < 0.2] = float("-inf")
            x[:, 0] = 0.0
        x, y = x.to(dt), y.to(dt)
        lab = torch.randint(0, V, (R,), generator=g)
        lab[torch.rand(R, generator=g) < 0.2] = -100
        print(f"[random row stats] seed={seed} {dt} R={R} V={V}", flush=True)
        st = row_stats(x.cuda(), lab.cuda(), y.cuda(), entropy=True, lse=True)
        torch.cuda.synchronize()
        assert _close(st.logprob, L.token_logprobs_from_logits(x, lab), 2e-5)[0], seed
        assert _close(st.entropy, L.entropy_from_logits(x), 2e-5)[0], seed
        assert _close(st.kl, L.kl_full_distribution(x, y), 2e-5)[0], seed
        assert _close(st.lse, L.logsumexp(x), 2e-5, 1e-6)[0], seed

"""Cases of the randomized sampling sweep that once came out MISMATCH,
rebuilt from their seeds and sampled on the GPU (MI355X)."""

import pytest
import torch

from tests.helpers import run_sweep_case

pytestmark = pytest.mark.gpu


def test_sweep_seed_71183_f16_top_p_after_an_open_min_p_boundary():
    """float16, V=151936, soft-cap 5 (8 rows).  Row 7's min-p boundary value
    lies 0.0012 float16-subnormal units from a rounding midpoint; the kernel
    rounds it down (removing its 65 members) where torch rounds it up, and the
    top-p cut inside a tied group of 535 then keeps 276 members against the
    oracle's 281.  Correct on the kernel's survivor set; every row must
    classify without MISMATCH and row 7 must keep exactly 276."""
    w, ok_rows, st, summ, verdicts, toks, keep = run_sweep_case(71183)
    print(f"seed 71183: status {st.tolist()} {summ}", flush=True)
    assert summ["MISMATCH"] == 0, [v.details[:3] for v in verdicts if not v.ok]
    assert 7 in ok_rows
    from oracle import sampler_oracle as O

    b = 7
    y = O.pre_filter_values(w.logits[b][None], float(w.temperature[b]), 1.0, None, w.softcap)[0]
    grp = torch.nonzero(y == 7.04296875).flatten()
    assert grp.numel() == 535
    assert int(keep[ok_rows.index(b)][grp].sum()) == 276


def test_sweep_seed_202175_f32_top_p_over_soft_capped_top_k_survivors():
    """float32, V=151936, soft-cap 5 over logits near 25 (8 rows).  Row 2
    (top-k 1000, top-p 0.9): three elements tie at the K-th value in the
    oracle, and the kernel's soft-cap puts one of them (index 74521) a unit
    lower, so its top-k keeps 1001 and its top-p cut 901 where the oracle
    keeps 1002 and 902.  Every row must classify without MISMATCH, and row 2
    must keep exactly the oracle's 901 largest values."""
    w, ok_rows, st, summ, verdicts, toks, keep = run_sweep_case(202175)
    print(f"seed 202175: status {st.tolist()} {summ}", flush=True)
    assert summ["MISMATCH"] == 0, [v.details[:3] for v in verdicts if not v.ok]
    assert 2 in ok_rows
    from oracle import sampler_oracle as O
    from tests.helpers import row_params

    p = row_params(w, 2)
    y = O.pre_filter_values(w.logits[2][None], p.temperature, p.repetition_penalty, p.history, w.softcap)[0]
    order = torch.sort(y, descending=True, stable=True).indices
    want = torch.zeros_like(keep[0])
    want[order[:901]] = True
    assert torch.equal(keep[ok_rows.index(2)], want)


def test_sweep_seed_401310_f32_top_p_next_to_the_soft_cap():
    """float32, V=151936, soft-cap 5, x ~ N(0, 60^2) (8 rows).  Row 0 (T 1.5,
    top-p 0.5, min-p 0.3): 34524 values sit at the cap and the top-p cut
    falls inside the group one unit below it.  The two smallest capped
    inputs (45.0543, 45.0545, indices 24710 and 29445) have tanh(x / 5) next
    to the midpoint between 1 and the float below it; the kernel rounds both
    down, they join the cut group, one lands past the cut and the token
    moves.  The kernel's mask and token must be the oracle's filters and
    draw on the kernel's own unfiltered values (within 8 units of the
    oracle's), so every row classifies without MISMATCH."""
    from oracle import sampler_oracle as O
    from tests.helpers import row_params, unfiltered_values

    w, ok_rows, st, summ, verdicts, toks, keep = run_sweep_case(401310)
    print(f"seed 401310: status {st.tolist()} {summ}", flush=True)
    assert summ["MISMATCH"] == 0, [v.details[:3] for v in verdicts if not v.ok]
    assert 0 in ok_rows
    wd = w.to("cuda")
    kw = wd.kwargs()
    kw.pop("uniforms")
    allv = unfiltered_values(wd.logits, kw).cpu()
    p = row_params(w, 0)
    y = O.pre_filter_values(w.logits[0][None], p.temperature, p.repetition_penalty, None, w.softcap)[0]
    # the two values below the cap on the kernel, at the cap in the oracle
    assert torch.equal(torch.nonzero((y == y.max()) & (allv[0] < y.max())).flatten(),
                       torch.tensor([24710, 29445]))
    st_ = allv[0][None].clone()
    st_ = O._min_p(st_, p.min_p)
    st_ = O._top_p(st_, p.top_p, True)
    assert torch.equal(keep[ok_rows.index(0)], ~torch.isneginf(st_[0]))
    assert int(toks[0]) == O.select_token(st_[0], float(w.uniforms[0]), p.temperature)

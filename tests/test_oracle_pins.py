"""Pins of the CPU oracle (oracle/sampler_oracle.py) against facts that do not
come from the oracle itself: numpy float32 closed forms, textbook selection,
brute force over tiny vocabularies, constructed cases whose answer is fixed by
the arithmetic, invariants, and a chi-square test of the draw.

Each check is chosen so that a plausible mistake in the restatement of
nanoserve/scheduler/sampler.py:28-89 fails it:

* penalty: multiply-by-reciprocal, float64 penalty, sign mix-up, applying a
  duplicated history id twice (sampler.py:31-38);
* temperature: the t -> max(t, 1e-6) / 1.0 mapping, greedy flag (:40-51);
* top-k: strict instead of >= comparison, k-th from the wrong end (:53-58);
* top-p: dropping the crossing token, >= instead of >, float32 accumulation
  of the cumulative sum, tie order at the cut (:60-73);
* softmax, NaN guard (:75-80), first-index argmax (:82-83), inverse-CDF draw.
"""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import sampler_oracle as O

F32 = np.float32


def run(rows, t=1.0, k=-1, p=1.0, pen=1.0, hist=None, u=0.5):
    rows = np.asarray(rows, dtype=np.float32)
    if rows.ndim == 1:
        rows = rows[None]
    B = rows.shape[0]
    bc = lambda v: [v] * B if np.isscalar(v) else list(v)
    hist = hist if hist is not None else [[] for _ in range(B)]
    return O.sample(rows, bc(t), bc(k), bc(p), bc(pen), hist, np.asarray(bc(u), dtype=np.float32))


# ----------------------------------------------------------------- penalty
def test_penalty_closed_form_float32():
    rng = np.random.default_rng(1)
    x = rng.normal(0, 3, size=4096).astype(F32)
    ids = np.arange(0, 4096, 3)
    r = run(x, pen=1.1, hist=[ids.tolist()])
    want = x.copy()
    pv = F32(1.1)
    sel = x[ids]
    want[ids] = np.where(sel < 0, sel * pv, sel / pv)
    got = r.penalized[0].numpy()
    assert np.array_equal(got.view(np.int32), want.view(np.int32))
    # the distinguishing facts: a reciprocal multiply and a float64 penalty both differ somewhere
    pos = sel[sel > 0]
    assert np.any(pos * (F32(1) / pv) != pos / pv)
    assert np.any((pos.astype(np.float64) / 1.1).astype(F32) != pos / pv)


def test_penalty_set_semantics_and_untouched_rows():
    x = np.array([2.0, -2.0, 4.0, -4.0, 1.0], dtype=F32)
    r = run(x, pen=2.0, hist=[[0, 0, 0, 1, 1]])
    # a duplicated id is penalized once: the gather happens before the scatter
    assert r.penalized[0].tolist() == [1.0, -4.0, 4.0, -4.0, 1.0]
    # penalty 1.0 and empty histories leave the row alone (sampler.py:33)
    assert run(x, pen=1.0, hist=[[0, 1]]).penalized[0].tolist() == x.tolist()
    assert run(x, pen=2.0, hist=[[]]).penalized[0].tolist() == x.tolist()
    # penalty below 1 boosts: division of a positive logit by 0.5 doubles it
    assert run(x, pen=0.5, hist=[[2, 3]]).penalized[0].tolist() == [2.0, -2.0, 8.0, -2.0, 1.0]


# ------------------------------------------------------------- temperature
def test_temperature_mapping_and_division():
    x = np.linspace(-5, 5, 101, dtype=F32)
    for t, teff in [(0.7, 0.7), (1.3, 1.3), (1e-9, 1e-6), (-2.0, 1.0), (0.0, 1.0)]:
        r = run(x, t=t, u=0.3)
        want = x / F32(teff)
        assert np.array_equal(r.scaled[0].numpy().view(np.int32), want.view(np.int32)), t
        assert bool(r.greedy[0]) == (t == 0.0)
    assert O.effective_temperature(0.0) == 1.0 and O.effective_temperature(-1.0) == 1.0
    assert O.effective_temperature(1e-9) == 1e-6


# ------------------------------------------------------------------- top-k
def test_topk_keeps_ties_at_threshold():
    r = run([5.0, 4.0, 4.0, 4.0, 3.0], k=2)
    assert float(r.topk_thr[0]) == 4.0
    assert int(r.n_kept_topk[0]) == 4
    assert np.isfinite(r.masked[0].numpy()).tolist() == [True, True, True, True, False]


def test_topk_against_partition():
    rng = np.random.default_rng(2)
    for k in (1, 7, 50, 999):
        x = rng.normal(0, 2.5, size=5000).astype(F32)
        x[rng.choice(5000, 40)] = x[0]  # ties
        r = run(x, k=k, t=0.8, u=0.1)
        y = x / F32(0.8)
        thr = np.partition(y, len(y) - k)[len(y) - k]
        assert float(r.topk_thr[0]) == float(thr)
        kept = np.isfinite(r.masked[0].numpy())
        assert kept.sum() >= k
        assert np.array_equal(kept, y >= thr)
        if (~kept).any():
            assert y[kept].min() > y[~kept].max()


def test_topk_off_values():
    x = np.arange(10, dtype=F32)
    for k in (0, -1, 10, 11):
        r = run(x, k=k)
        assert int(r.n_kept_topk[0]) == 10 and np.isnan(r.topk_thr[0])


# ------------------------------------------------------------------- top-p
def brute_topp(x, p):
    """Shortest prefix of the (value desc, id asc) order whose exactly summed
    float32 sorted probabilities exceed float32(p), computed with Fractions."""
    x = np.asarray(x, dtype=np.float64)
    order = sorted(range(len(x)), key=lambda i: (-x[i], i))
    e = np.exp(x[order] - x.max())
    q = (e / e.sum()).astype(F32)
    p32 = Fraction(float(F32(p)))
    run_ = Fraction(0)
    for j in range(len(order)):
        run_ += Fraction(float(q[j]))
        # the reference keeps position j+1 only while the float32-rounded prefix is <= p
        if Fraction(float(F32(float(run_)))) > p32:
            return set(order[:j + 1])
    return set(order)


@pytest.mark.parametrize("seed", range(40))
def test_topp_brute_force_tiny_vocab(seed):
    rng = np.random.default_rng(100 + seed)
    V = int(rng.integers(2, 12))
    x = rng.normal(0, 2, size=V).astype(F32)
    if seed % 3 == 0:
        x[rng.integers(0, V)] = x[0]
    p = float(rng.choice([0.0, 0.3, 0.5, 0.9, 0.95, 0.999]))
    r = run(x, p=p, u=0.5)
    kept = set(np.flatnonzero(np.isfinite(r.masked[0].numpy())).tolist())
    assert kept == brute_topp(x, p)


def test_topp_keeps_crossing_token_and_is_strict():
    # probabilities exactly 0.5, 0.25, 0.25
    x = np.log(np.array([0.5, 0.25, 0.25])).astype(F32)
    r = run(x, p=0.5)
    assert r.masked[0].numpy()[2] == -np.inf and np.isfinite(r.masked[0].numpy()[:2]).all()
    assert int(r.n_kept[0]) == 2  # c0 = 0.5 is not > 0.5, so the second token survives
    r = run(x, p=0.49)
    assert int(r.n_kept[0]) == 1  # c0 = 0.5 > 0.49: only the head survives
    r = run(x, p=0.0)
    assert int(r.n_kept[0]) == 1  # top_p <= 0 keeps exactly one token


def test_topp_tie_order_lower_id_first():
    r = run([1.0, 1.0, 1.0, 1.0], p=0.3)
    assert np.isfinite(r.masked[0].numpy()).tolist() == [True, True, False, False]
    assert bool(r.topp_tie_straddle[0])


def test_topp_cumsum_accumulates_in_float64():
    # head mass 1 - 64*eps, then 64 tokens of mass eps = 2^-26: a float32 accumulator
    # never moves past 1 - 64 eps (each add is below half an ulp), a float64 one does.
    eps = 2.0 ** -26
    n_tiny = 64
    probs = np.array([0.6, 0.4 - n_tiny * eps] + [eps] * n_tiny, dtype=np.float64)
    x = np.log(probs).astype(F32)
    q = O.softmax_exact(torch.from_numpy(x)).numpy()
    order = np.argsort(-x, kind="stable")
    qs = q[order]
    # float32 running sum stalls; float64 running sum rounded per prefix keeps climbing
    acc32 = F32(0)
    pre32 = []
    for v in qs:
        acc32 = F32(acc32 + v)
        pre32.append(acc32)
    pre64 = np.cumsum(qs.astype(np.float64)).astype(F32)
    top_p = float(pre64[40])  # a prefix value reached only by the float64 accumulation
    assert top_p > max(pre32[:-1]) or pre32.count(pre32[-1]) > 1
    r = run(x, p=top_p)
    want = brute_topp(x, top_p)
    kept = set(np.flatnonzero(np.isfinite(r.masked[0].numpy())).tolist())
    assert kept == want
    assert len(want) < len(x)


def test_topp_exact_ties_have_no_zone():
    """Survivors that all tie have probabilities 1/n in any arithmetic, so the cut is fixed:
    two tied tokens at top_p 0.5 give prefixes 0.5 and 1.0, 0.5 is not > 0.5, both stay
    (Fraction brute force); a 1e-6 zone would have admitted keeping one."""
    x = np.array([2.0, 7.0, 7.0, 1.0, -3.0], dtype=F32)
    r = run(x, k=1, p=0.5, t=1.3, u=0.75)
    assert brute_topp(np.where(x == 7.0, x, -np.inf), 0.5) == {1, 2}
    assert r.alt_kept[0].tolist() == [2] and int(r.n_kept[0]) == 2
    assert r.probs[0].numpy()[[1, 2]].tolist() == [0.5, 0.5]
    assert r.allowed_ids[0].tolist() == [2]                  # u = 0.75 lies inside token 2's interval
    # four ties at top_p 0.5: prefixes 0.25, 0.5, 0.75; the crossing token (prefix 0.5 is not
    # > 0.5) stays, so three are kept, and no alternative either
    r = run([3.0, 3.0, 3.0, 3.0], p=0.5, u=0.1)
    assert brute_topp([3.0] * 4, 0.5) == {0, 1, 2}
    assert r.alt_kept[0].tolist() == [3]


def _closed_form_alternative(y, n_keep, u):
    """Probabilities and allowed ids of keeping the n_keep largest values (id ascending on
    ties), in float64 with math.fsum, and the inverse-CDF candidates within 1e-6 of u."""
    order = sorted(range(len(y)), key=lambda i: (-float(y[i]), i))[:n_keep]
    e = np.zeros(len(y))
    m = max(float(y[i]) for i in order)
    for i in order:
        e[i] = math.exp(float(y[i]) - m)
    q = (e / math.fsum(e)).astype(F32)
    c = np.cumsum(q.astype(np.float64))
    ok = [t for t in order if (c[t - 1] if t else 0.0) - 1e-6 <= u < c[t] + 1e-6]
    return q, ok


def test_topp_admissible_cuts_closed_form():
    """A prefix sum within 1e-6 of top_p makes two cuts admissible.  Each alternative's
    probabilities are the float64 softmax over its own kept set (closed form, not the oracle's
    code) and its allowed ids the CDF intervals within 1e-6 of u; a cut outside the zone is
    not admissible."""
    # probabilities 0.5, 0.3, 0.2 (sorted ids 0, 2, 1): prefixes 0.5, 0.8, 1.0
    x = np.log(np.array([0.5, 0.2, 0.3], dtype=np.float64)).astype(F32)
    q = O.softmax_exact(torch.from_numpy(x)).numpy()
    top_p = float(np.float32(np.float64(q[0]) + np.float64(q[2])) - np.float32(4e-7))  # 0.8 - 4e-7
    for u in (0.1, 0.49, 0.6, 0.95):
        r = run(x, p=top_p, u=u)
        assert r.alt_kept[0].tolist() == [2, 3], r.alt_kept[0]
        assert r.alternative(0, 1) is None and r.alternative(0, 4) is None
        for n_keep in (2, 3):
            probs, allowed = r.alternative(0, n_keep)
            qc, ok = _closed_form_alternative(x.astype(np.float64), n_keep, u)
            np.testing.assert_allclose(probs.numpy(), qc, rtol=1e-6, atol=0)
            assert sorted(allowed.tolist()) == sorted(ok), (u, n_keep, allowed, ok)
        assert set(r.allowed_ids[0].tolist()) == set(r.alternative(0, 2)[1].tolist()) | set(
            r.alternative(0, 3)[1].tolist())
    # away from the zone: one alternative, and it is the oracle's own result
    r = run(x, p=0.7, u=0.6)
    assert r.alt_kept[0].tolist() == [int(r.n_kept[0])] == [2]


def test_penalty_reciprocal_rounding_closed_form():
    """penalty_rounding="reciprocal": positive logits times float32(1 / p), the float64
    reciprocal rounded once (torch on a GPU for ``score / p``), negative ones times p as before;
    it differs from the division, and for p = 1.1 from the float32 reciprocal 1 / float32(p)."""
    rng = np.random.default_rng(11)
    x = rng.normal(0, 3, size=8192).astype(F32)
    ids = np.arange(0, 8192, 2)
    for pv in (1.1, 1.2, 0.8, 1.3):
        rows = O.sample(x[None], [1.0], [-1], [1.0], [pv], [ids.tolist()], np.array([0.5], dtype=F32),
                        penalty_rounding="reciprocal")
        want = x.copy()
        sel = x[ids]
        want[ids] = np.where(sel < 0, sel * F32(pv), sel * F32(1.0 / pv))
        assert np.array_equal(rows.penalized[0].numpy().view(np.int32), want.view(np.int32)), pv
        div = O.sample(x[None], [1.0], [-1], [1.0], [pv], [ids.tolist()], np.array([0.5], dtype=F32))
        assert not torch.equal(rows.penalized, div.penalized), pv
        if pv == 1.1:
            assert F32(1.0 / pv) != F32(1) / F32(pv)
            single = x[ids] * (F32(1) / F32(pv))
            assert np.any(single[x[ids] > 0] != rows.penalized[0].numpy()[ids][x[ids] > 0])
    with pytest.raises(ValueError):
        O.sample(x[None], [1.0], [-1], [1.0], [1.1], [ids.tolist()], np.array([0.5], dtype=F32),
                 penalty_rounding="fp64")


# ------------------------------------------------- softmax, NaN, argmax, draw
def test_softmax_closed_form_and_masked_zeros():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 3, size=3000).astype(F32)
    r = run(x, k=100, t=1.3, u=0.2)
    y = (x / F32(1.3)).astype(np.float64)
    keep = np.isfinite(r.masked[0].numpy())
    e = np.where(keep, np.exp(y - y.max()), 0.0)
    want = e / math.fsum(e)
    got = r.probs[0].numpy().astype(np.float64)
    assert np.all(got[~keep] == 0.0)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=0)


def test_nan_guard_uniform_row():
    x = np.zeros(16, dtype=F32)
    x[3] = np.nan
    r = run(x, t=0.9, u=0.51)
    assert bool(r.nan_row[0])
    assert np.all(r.probs[0].numpy() == F32(1.0 / 16))
    assert int(r.ids[0]) == 8  # floor(0.51 * 16) in the uniform inverse CDF


def test_greedy_first_index_and_ignores_uniform():
    x = np.array([1.0, 3.0, 3.0, 2.0], dtype=F32)
    for u in (0.0, 0.5, 0.999):
        r = run(x, t=0.0, u=u, k=3, p=0.5)
        assert int(r.ids[0]) == 1
    # the penalty can move the argmax
    r = run(x, t=0.0, pen=2.0, hist=[[1]])
    assert int(r.ids[0]) == 2


def test_inverse_cdf_grid():
    x = np.log(np.array([0.1, 0.2, 0.3, 0.4])).astype(F32)
    q = O.softmax_exact(torch.from_numpy(x)).numpy().astype(np.float64)
    C = np.cumsum(q)
    for u in np.linspace(0, 0.999, 97, dtype=F32):
        r = run(x, u=float(u))
        want = next(i for i in range(4) if C[i] > float(u))
        assert int(r.ids[0]) == want


def test_inverse_cdf_is_strict_and_skips_masked_tokens():
    # probabilities exactly 0.5, 0.25, 0.25: a uniform equal to C_0 = 0.5 picks token 1
    x = np.log(np.array([0.5, 0.25, 0.25])).astype(F32)
    assert int(run(x, u=0.5).ids[0]) == 1
    assert int(run(x, u=0.0).ids[0]) == 0
    # a masked (zero-probability) token is never drawn, even when u equals the mass before it
    r = run(np.array([1.0, -3.0, 1.0], dtype=F32), k=2, u=0.5)
    assert float(r.probs[0, 1]) == 0.0 and int(r.ids[0]) == 2


def test_draw_chi_square():
    rng = np.random.default_rng(4)
    V = 12
    x = rng.normal(0, 1, size=V).astype(F32)
    n = 4000
    us = rng.random(n, dtype=np.float32)
    r = O.sample(np.repeat(x[None], n, 0), [1.0] * n, [-1] * n, [1.0] * n, [1.0] * n, [[]] * n, us)
    counts = np.bincount(r.ids, minlength=V)
    expect = r.probs[0].numpy().astype(np.float64) * n
    chi2 = float(((counts - expect) ** 2 / expect).sum())
    assert chi2 < 40.0  # 11 degrees of freedom: p ~ 4e-5 at 40


# --------------------------------------------------------------- invariants
@settings(max_examples=60, deadline=None)
@given(seed=st.integers(0, 2**31 - 1), V=st.integers(2, 400), k=st.integers(-1, 450),
       p=st.sampled_from([0.0, 0.3, 0.5, 0.9, 0.95, 1.0]), t=st.sampled_from([0.0, 0.5, 1.0, 1.7]),
       pen=st.sampled_from([1.0, 1.2, 0.8]))
def test_invariants(seed, V, k, p, t, pen):
    rng = np.random.default_rng(seed)
    x = np.round(rng.normal(0, 2, size=V), 1).astype(F32)  # rounding makes ties common
    hist = rng.integers(0, V, size=int(rng.integers(0, 20))).tolist()
    u = F32(rng.random())
    r = run(x, t=t, k=k, p=p, pen=pen, hist=[hist], u=float(u))
    masked = r.masked[0].numpy()
    kept = np.isfinite(masked)
    y = r.scaled[0].numpy()
    amax = int(np.argmax(y))
    assert kept[amax]                                   # the maximum always survives
    if 0 < k < V:
        assert int(r.n_kept_topk[0]) >= k
    if p < 1.0 and kept.sum() < (np.isfinite(y)).sum():
        assert r.probs[0].numpy()[kept].sum() > 0       # nonempty nucleus
    pr = r.probs[0].numpy().astype(np.float64)
    assert abs(pr.sum() - 1.0) < 1e-5
    assert np.all(pr[~kept] == 0.0)
    if t == 0.0:
        assert int(r.ids[0]) == amax
    else:
        assert kept[int(r.ids[0])]
    # duplicate history ids: same penalized row as the deduplicated history
    r2 = run(x, t=t, k=k, p=p, pen=pen, hist=[sorted(set(hist))], u=float(u))
    assert torch.equal(r.penalized, r2.penalized) and int(r.ids[0]) == int(r2.ids[0])


def test_baseline_restatement_draws_inside_the_kept_set():
    """The timed CPU baseline (the reference's op sequence with torch.multinomial)
    samples only tokens of the oracle's kept set and returns the argmax for greedy rows."""
    rng = np.random.default_rng(5)
    B, V = 12, 3000
    x = rng.normal(0, 2.5, size=(B, V)).astype(F32)
    t = [0.0, 0.7, 1.0, 1.3] * 3
    k = [0, 1, 20, 50] * 3
    p = [1.0, 0.95, 0.5] * 4
    pen = [1.0, 1.2] * 6
    hist = [rng.integers(0, V, size=50).tolist() for _ in range(B)]
    r = O.sample(x, t, k, p, pen, hist, np.full(B, 0.5, dtype=F32))
    g = torch.Generator()
    for s in range(5):
        g.manual_seed(s)
        ids = O.reference_restatement_multinomial(torch.from_numpy(x), t, k, p, pen, hist, generator=g).numpy()
        for i in range(B):
            if r.greedy[i]:
                assert ids[i] == r.ids[i]
            else:
                assert np.isfinite(r.masked[i, ids[i]].item()), (i, ids[i])

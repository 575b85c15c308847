"""Pins the oracle's sampling restatement (orc_sample_logits, orc_repetition_penalty;
decoder.rs:878-1020) before it checks the device sampler.

  greedy        numpy argmax (first index); NaN skipped, +inf taken; the
                temperature / top_k conditions of decoder.rs:919-931
  distribution  the fraction of a fine grid of u that lands on each token equals
                a float64 numpy softmax over the top-k with the nucleus cut
  nucleus rule  the reference's cut (drop items whose preceding mass already
                exceeds top_p) on hand-made distributions
  order / ties  u = 0 takes the largest (lowest index among equal values)
  penalty       closed form: distinct tokens once, / when positive, * otherwise
"""
import numpy as np
import pytest

from oracle import oracle as O


def test_greedy_cases():
    g = np.random.default_rng(1)
    lg = g.standard_normal(1000).astype(np.float32)
    want = int(np.argmax(lg))
    for t, k in [(0.0, 40), (-1.0, 40), (float("nan"), 40), (float("inf"), 40), (0.7, 1)]:
        assert O.sample_logits(lg, t, k, 1.0, 0.5)[0] == want
    lg2 = lg.copy()
    lg2[3] = np.nan
    lg2[700] = np.nanmax(lg2) + 1
    assert O.sample_logits(lg2, 0.0, 40, 1.0, 0.0)[0] == 700
    lg2[9] = np.inf
    assert O.sample_logits(lg2, 0.0, 40, 1.0, 0.0)[0] == 9
    ties = np.zeros(50, np.float32)
    assert O.sample_logits(ties, 0.0, 5, 1.0, 0.0)[0] == 0


def expected_probs(lg, T, k, top_p):
    lg = np.where(np.isfinite(lg), lg, -np.inf).astype(np.float64)
    order = sorted(range(lg.size), key=lambda i: (-lg[i], i))[:k]
    v = lg[order]
    p = np.exp((v - v[0]) / T)
    if 0 < top_p < 1 and k > 1:
        q = p / p.sum()
        before = np.concatenate([[0.0], np.cumsum(q)[:-1]])
        keep = before <= top_p
        p = p[keep]
        order = [o for o, kk in zip(order, keep) if kk]
    return dict(zip(order, p / p.sum()))


@pytest.mark.parametrize("T,k,top_p", [(0.7, 40, 1.0), (1.0, 10, 0.9), (1.5, 128, 0.5),
                                       (0.3, 5, 0.0)])
def test_distribution_over_u(T, k, top_p):
    g = np.random.default_rng(int(T * 10) + k)
    lg = (g.standard_normal(500) * 2).astype(np.float32)
    lg[17] = np.nan
    lg[18] = -np.inf
    want = expected_probs(lg, T, k, top_p)
    grid = (np.arange(20000) + 0.5) / 20000
    counts = {}
    for u in grid:
        tok, kept = O.sample_logits(lg, T, k, top_p, u)
        counts[tok] = counts.get(tok, 0) + 1
    assert kept == k
    assert set(counts) <= set(want)
    for tok, p in want.items():
        assert abs(counts.get(tok, 0) / grid.size - p) < 2e-4, (tok, p)


def test_nucleus_rule():
    probs = np.array([0.5, 0.3, 0.2])
    lg = np.log(probs).astype(np.float32)
    # preceding mass 0, 0.5, 0.8: an item stays while the mass before it is <= top_p
    for top_p, want in [(0.55, {0, 1}), (0.49, {0}), (0.85, {0, 1, 2}), (0.79, {0, 1})]:
        toks = {O.sample_logits(lg, 1.0, 3, top_p, u)[0] for u in np.linspace(0, 0.999, 200)}
        assert toks == want, top_p


def test_order_and_ties():
    lg = np.array([1.0, 3.0, 3.0, 2.0, 3.0], np.float32)
    assert O.sample_logits(lg, 1.0, 5, 1.0, 0.0)[0] == 1
    # k = 2 keeps the two lowest indices of the three tied maxima
    toks = {O.sample_logits(lg, 1.0, 2, 1.0, u)[0] for u in np.linspace(0, 0.999, 50)}
    assert toks == {1, 2}


def test_repetition_penalty_closed_form():
    lg = np.array([2.0, -1.0, 0.0, 4.0, -3.0], np.float32)
    out = O.repetition_penalty(lg, [0, 1, 0, 9, -1, 4, 1], 2.0)
    assert list(out) == [1.0, -2.0, 0.0, 4.0, -6.0]
    assert np.array_equal(O.repetition_penalty(lg, [0, 1], 1.0), lg)

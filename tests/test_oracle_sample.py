"""Pins the oracle's sampling restatement (orc_sample_logits, orc_repetition_penalty;
decoder.rs:878-1020) before it checks the device sampler.

  greedy        numpy argmax (first index); NaN past index 0 skipped, a NaN
                at index 0 kept (the reference's scan), +inf taken; the
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
    # decoder.rs:914-925 starts from logits[0] and compares with strict >: a NaN
    # there is never replaced, a NaN elsewhere never taken
    lg3 = lg.copy()
    lg3[0] = np.nan
    assert O.sample_logits(lg3, 0.0, 40, 1.0, 0.0)[0] == 0
    assert O.argmax(lg3) == 0


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


# ---------------------------------------------------------- speculative ---

def softmax64(row, T=1.0):
    r = np.where(np.isfinite(row), row, -np.inf).astype(np.float64) / T
    e = np.exp(r - r.max())
    return e / e.sum()


def test_speculative_accept_rules():
    """Closed forms of decoder.rs:608-726: a draft token the target rates at
    least as likely is always accepted; a rejection draws from the normalised
    max(0, p_t - p_d); all accepted draws the bonus from the last row."""
    g = np.random.default_rng(11)
    V, K = 50, 3
    rows = (g.standard_normal((K, V)) * 2).astype(np.float32)
    pt = [softmax64(r) for r in rows]
    draft = [int(np.argmax(p)) for p in pt]
    dp = np.zeros((K, V), np.float32)
    for i in range(K):
        dp[i, draft[i]] = np.float32(pt[i][draft[i]] * 0.5)   # p_t >= p_d: always accepted
    acc, _ = O.speculative_accept(rows, draft, dp, [0.999999] * (K + 1))
    assert acc == K
    # all accepted: the bonus distribution over u is the last row's softmax
    grid = (np.arange(4000) + 0.5) / 4000
    cnt = np.zeros(V)
    for uu in grid:
        cnt[O.speculative_accept(rows, draft, dp, [0.0] * K + [uu])[1]] += 1
    assert np.abs(cnt / grid.size - pt[-1]).max() < 1e-3
    # rejection at position 1: the bonus distribution is max(0, p_t - p_d)
    dp2 = np.full((K, V), 1.0 / V, np.float32)
    dp2[1, draft[1]] = 1.0                  # draft far more confident than the target
    c = np.maximum(pt[1] - dp2[1].astype(np.float64), 0)
    c /= c.sum()
    cnt = np.zeros(V)
    for uu in grid:
        a, b = O.speculative_accept(rows, draft, dp2, [0.0, 0.999999, uu])
        assert a == 1
        cnt[b] += 1
    assert np.abs(cnt / grid.size - c).max() < 1e-3
    # acceptance threshold p_t / p_d: u just above rejects, just below accepts
    ratio = pt[1][draft[1]] / (1.0 + 1e-12)
    assert O.speculative_accept(rows, draft, dp2, [0.0, ratio * 0.999, 0.5])[0] >= 2
    assert O.speculative_accept(rows, draft, dp2, [0.0, ratio * 1.001, 0.5])[0] == 1


def test_speculative_accept_nucleus_and_empty():
    probs = np.array([0.5, 0.3, 0.2])
    rows = np.log(probs).astype(np.float32)[None]
    dp = np.zeros((1, 3), np.float32)
    bon = {O.speculative_accept(rows, [0], dp, [0.0, uu], top_p=0.6)[1]
           for uu in np.linspace(0, 0.999, 100)}
    assert bon == {0, 1}
    assert O.speculative_accept(np.zeros((0, 7), np.float32), [], np.zeros(0, np.float32),
                                []) == (0, 6)

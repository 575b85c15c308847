"""The device sampler (tb_sample_logits) against the oracle's restatement of
apply_repetition_penalty + sample_logits (decoder.rs:878-1020), pinned in
tests/test_oracle_sample.py.  The draw u of (seed, counter) comes from the
library's generator (tb_sample_uniform); given u the token must be identical
for top_k <= 1024 (the list / select path sums the masses of its at most 1024
items in sequence, as the oracle does).  Past that the one-block path sums them
in a parallel order and the token must lie between the oracle's draws at
u -/+ 2e-3.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
import torchburn_amd as tb

pytestmark = pytest.mark.gpu


CASES = [
    # V, T, top_k, top_p, penalty
    (1000, 0.7, 40, 1.0, 1.0),
    (151936, 0.7, 40, 0.9, 1.1),
    (128256, 1.3, 128, 0.5, 1.0),
    (2048 * 3 + 5, 0.5, 2, 1.0, 1.2),
    (151936, 0.0, 40, 1.0, 1.0),       # greedy
    (151936, 0.9, 1, 1.0, 1.3),        # top_k 1 -> greedy after the penalty
    (5000, 1.0, 0, 1.0, 1.0),          # top_k 0 -> one candidate
    (300, 2.0, 128, 0.95, 1.5),
    (32000, 0.8, 128, 0.95, 1.1),      # fewer waves than k: every listed item competes
    (5000, 1.0, 100, 0.9, 1.0),        # lists too short for k: the exact select
    # top_k past the slice path: one block over the whole vocabulary
    (151936, 0.8, 500, 0.9, 1.1),
    (151936, 0.8, 512, 0.9, 1.0),
    (151936, 1.1, 1024, 0.95, 1.0),     # the largest k of the list / select path
    (32000, 0.9, 700, 0.9, 1.1),        # fewer waves than k, past 128
    (151936, 0.9, 1025, 0.9, 1.0),      # the first k of the one-block path
    (1, 0.8, 40, 0.9, 1.1),             # tiny vocabularies: empty waves, k clamped to V
    (3, 0.8, 2, 0.9, 1.1),
    (7, 1.0, 7, 1.0, 1.0),
    (2049, 0.8, 64, 0.9, 1.0),          # a second list block with one logit
    (65537, 0.9, 300, 0.95, 1.1),
    (128256, 1.0, 4096, 1.0, 1.0),
    (1000, 0.7, 1000, 0.95, 1.0),       # k == V
    (300, 2.0, 129, 1.0, 1.2),
    (5000, 0.5, 200000, 0.8, 1.0),      # k > V
    (151936, 1.0, 151936, 0.5, 1.0),    # the whole vocabulary, nucleus cut
]


@pytest.mark.parametrize("V,T,k,top_p,pen", CASES)
def test_sampler_matches_oracle(cuda, V, T, k, top_p, pen):
    print(f"case sample_logits V={V} T={T} top_k={k} top_p={top_p} penalty={pen}", flush=True)
    g = np.random.default_rng(V + k)
    for trial in range(7):
        lg = (g.standard_normal(V) * 3).astype(np.float32)
        if trial == 1:
            lg[g.integers(0, V, 20)] = np.nan
            lg[g.integers(0, V, 5)] = -np.inf
        if trial == 2:
            lg[:] = np.round(lg)                  # many ties
        if trial == 3:
            lg[:] = 0.0                           # all equal
        if trial == 4:
            lg[0] = np.nan                        # greedy keeps index 0 (decoder.rs:914-925)
            if V > 1:
                lg[g.integers(1, V, 3)] = np.nan
        recent = list(g.integers(0, V, 30)) + [V + 5, -1]
        seed, counter = int(g.integers(0, 2 ** 63)), int(g.integers(0, 1000))
        tok, u = tb.sample_logits(torch.from_numpy(lg).to(cuda), T, k, top_p, pen, recent,
                                  seed=seed, counter=counter, return_u=True)
        greedy = not np.isfinite(T) or T <= 0 or k == 1
        uu = tb.sample_uniform(seed, counter)
        if not greedy and max(1, min(k, V)) > 1:
            assert u == uu
        else:
            assert u == -1.0
        pl = O.repetition_penalty(lg, recent, pen)
        ref, _ = O.sample_logits(pl, T, k, top_p, uu)
        if greedy or k <= 1024 or tok == ref:
            assert tok == ref, (trial, tok, ref)
            continue
        # top_k > 1024: the masses are summed in a parallel order, and over tens
        # of thousands of f32 terms that moves the nucleus cut and the draw
        # point by up to ~1e-4 of the mass.  The draw is monotone in u over the
        # sorted order (value descending, index ascending), so the token must
        # lie between the oracle's draws at u -/+ 2e-3.
        key = np.where(np.isfinite(pl), pl, -np.inf)
        order = np.lexsort((np.arange(V), -key.astype(np.float64)))
        pos = np.empty(V, np.int64)
        pos[order] = np.arange(V)
        lo, _ = O.sample_logits(pl, T, k, top_p, max(0.0, uu - 2e-3))
        hi, _ = O.sample_logits(pl, T, k, top_p, min(1.0 - 2 ** -24, uu + 2e-3))
        assert pos[lo] <= pos[tok] <= pos[hi], (trial, tok, ref, pos[lo], pos[tok], pos[hi])


def test_sampler_leaves_logits_and_limits(cuda):
    lg = torch.randn(1000, device=cuda)
    before = lg.clone()
    tb.sample_logits(lg, 0.7, 40, 1.0, 1.5, [1, 2, 3])
    assert torch.equal(lg, before)
    tb.sample_logits(lg, 0.7, 129)   # any top_k on the device
    with pytest.raises(tb.UnsupportedOpError, match="vocabulary"):
        tb.sample_logits(torch.randn(262145, device=cuda), 0.7, 40)


def test_sampler_seed_reproducible_and_distribution(cuda):
    V = 64
    g = np.random.default_rng(5)
    lg = (g.standard_normal(V) * 1.5).astype(np.float32)
    t = torch.from_numpy(lg).to(cuda)
    a = [tb.sample_logits(t, 1.0, 16, 1.0, seed=7, counter=i) for i in range(400)]
    b = [tb.sample_logits(t, 1.0, 16, 1.0, seed=7, counter=i) for i in range(400)]
    assert a == b
    order = sorted(range(V), key=lambda i: (-lg[i], i))[:16]
    p = np.exp(lg[order].astype(np.float64) - lg[order[0]])
    p /= p.sum()
    freq = np.array([a.count(o) for o in order]) / len(a)
    assert set(a) <= set(order)
    assert np.abs(freq - p).max() < 0.08


def _wave_ids(V, b, w):
    """The ids one wave of the list kernel holds: runs of 16 ids, block b of
    nb takes runs b, b + nb, ..., and wave w the ids = w (mod 4) of each."""
    nb = (V + 2047) // 2048
    ids = [16 * (b + nb * ((l >> 2) + 16 * i)) + 4 * (l & 3) + w
           for l in range(64) for i in range(8)]
    return np.array([i for i in ids if i < V])


@pytest.mark.parametrize("kind", ["low_ids", "bands", "few_finite", "finite_below_k", "one_wave"])
def test_sampler_wave_list_edges(cuda, kind):
    """Logits laid out against the list kernel's waves: top tokens crowded into
    the lowest ids (waves re-read), into whole waves by descending bands (more
    candidates than the select block holds: the exact select), or finite in a
    few places only; tokens identical to the oracle for top_k <= 128."""
    print(f"case wave lists {kind}", flush=True)
    V = 151936
    g = np.random.default_rng(len(kind))
    for k in (40, 128, 600):
        lg = g.standard_normal(V).astype(np.float32)
        if kind == "low_ids":
            lg[:94] += 10.0
        elif kind == "bands":
            for n in range(16):
                ids = _wave_ids(V, n // 4, n % 4)
                lg[ids] = 10 + 2 * n + g.random(len(ids)).astype(np.float32)
        elif kind == "few_finite":
            keep = g.choice(V, 300, replace=False)
            lg[np.setdiff1d(np.arange(V), keep)] = -np.inf
        elif kind == "finite_below_k":
            keep = g.choice(V, 50, replace=False)
            lg[np.setdiff1d(np.arange(V), keep)] = -np.inf
        else:
            ids = _wave_ids(V, 3, 1)
            lg[ids] += 8.0
        for c in range(3):
            u = tb.sample_uniform(11, c)
            tok = tb.sample_logits(torch.from_numpy(lg).to(cuda), 0.9, k, 0.95, seed=11,
                                   counter=c)
            ref, _ = O.sample_logits(lg, 0.9, k, 0.95, u)
            assert tok == ref, (kind, k, c, tok, ref)

"""The library's host-side speculative acceptance (tb_speculative_accept_rows,
decoder.rs:608-726) against the oracle, given the same target rows, draft
probabilities and uniforms; no GPU (pure host code in libtbhip.so)."""
import numpy as np
import pytest

from oracle import oracle as O
from torchburn_amd import decoder as D


@pytest.mark.parametrize("V,K,T,top_p", [(300, 4, 1.0, 1.0), (1000, 2, 0.7, 0.9),
                                         (64, 6, 1.5, 0.5)])
def test_acceptance_matches_oracle(V, K, T, top_p):
    g = np.random.default_rng(V + K)
    for trial in range(30):
        rows = (g.standard_normal((K, V)) * 2).astype(np.float32)
        if trial % 5 == 1:
            rows[0, 3] = np.nan
            rows[-1, 7] = -np.inf
        dp = g.random((K, V)).astype(np.float32) ** 4
        dp /= dp.sum(1, keepdims=True)
        draft = [int(g.integers(0, V)) if trial % 3 else int(np.argmax(r)) for r in rows]
        u = list(g.random(K + 1))
        assert D.speculative_accept_rows(rows, draft, dp, u, T, top_p) == \
            O.speculative_accept(rows, draft, dp, u, T, top_p)


def test_spec_uniform_stream():
    u = [D.spec_uniform(9, i) for i in range(200)]
    assert all(0.0 <= x < 1.0 for x in u) and len(set(u)) == 200
    assert D.spec_uniform(9, 3) == u[3]

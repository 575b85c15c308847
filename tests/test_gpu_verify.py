"""verify_tokens as one batched forward and speculative_accept on the GPU decoder,
against the oracle's step-by-step decoder (decoder.rs:565-727).

verify: every position's logits within 2e-4 (max|d| / max|ref|) of the oracle's
steps, and the cache it leaves drives the next step identically.
speculative_accept: the decoder's result equals the oracle's acceptance over
the oracle's own target rows with the same uniforms (tb_spec_uniform stream).
"""
import numpy as np
import pytest

from oracle import oracle as O
from torchburn_amd import synth
from torchburn_amd.decoder import decoder_from_weights, spec_uniform

pytestmark = pytest.mark.gpu


def small(**kw):
    cfg = dict(num_layers=2, hidden=256, intermediate=512, num_heads=4, num_kv_heads=2,
               head_dim=64, vocab=1000, eps=1e-6, rope_theta=1e6, qkv_bias=True)
    cfg.update(kw)
    return cfg


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def make(cfg, wk, lk, max_seq=128, seed=41):
    w = synth.decoder_weights(cfg, seed, wk, lk, 32)
    ocfg = dict(num_layers=cfg["num_layers"], hidden=cfg["hidden"],
                intermediate=cfg["intermediate"], num_heads=cfg["num_heads"],
                num_kv_heads=cfg["num_kv_heads"], head_dim=cfg["head_dim"], vocab=cfg["vocab"],
                group_size=32, max_seq=max_seq, rope_theta=cfg["rope_theta"], eps=cfg["eps"],
                wkind=wk, lmkind=lk)
    return O.Decoder(w, ocfg), decoder_from_weights(w, cfg, group_size=32, max_seq_len=max_seq)


@pytest.mark.parametrize("wk,lk,n", [(4, 4, 5), (4, 32, 9), (4, 8, 2), (8, 8, 4), (4, 4, 1),
                                     (4, 4, 70)])
def test_verify_matches_oracle_steps(cuda, wk, lk, n):
    print(f"case verify_tokens wk={wk} lk={lk} n={n}", flush=True)
    ref, dec = make(small(), wk, lk)
    g = np.random.default_rng(n)
    pre = [int(t) for t in g.integers(0, 1000, 10)]
    for i, t in enumerate(pre):
        ref.step(t, i)
    dec.prefill_tokens(pre, 0)
    toks = [int(t) for t in g.integers(0, 1000, n)]
    rows = dec.verify_tokens(10, toks)
    want = [ref.step(t, 10 + i) for i, t in enumerate(toks)]
    err = max(rel(a, b) for a, b in zip(rows, want))
    print(f"verify rows rel err {err:.3g}", flush=True)
    assert len(rows) == n and err < 2e-4
    assert rel(dec.get_logits(), want[-1]) < 2e-4
    assert dec.kv_len() == 10 + n
    lg, am = dec._step(toks[-1], 10 + n, True)
    lo = ref.step(toks[-1], 10 + n)
    assert rel(lg, lo) < 2e-4 and am == O.argmax(lo)
    with pytest.raises(ValueError):
        dec.verify_tokens(126, [1, 2, 3])
    ref.close()
    dec.close()


@pytest.mark.parametrize("T,top_p", [(1.0, 1.0), (0.8, 0.9)])
def test_speculative_accept_matches_oracle(cuda, T, top_p):
    print(f"case speculative_accept T={T} top_p={top_p}", flush=True)
    V, K = 1000, 4
    g = np.random.default_rng(int(T * 10))
    outcomes = set()
    for trial in range(6):
        ref, dec = make(small(), 4, 4, seed=50 + trial)
        pre = [int(t) for t in g.integers(0, V, 12)]
        for i, t in enumerate(pre):
            ref.step(t, i)
        dec.prefill_tokens(pre, 0)
        # drafts: the target's own argmax path for some trials, random for others
        draft = [int(t) for t in g.integers(0, V, K)]
        dp = g.random((K, V)).astype(np.float32) ** 6
        dp /= dp.sum(1, keepdims=True)
        seed = 1000 + trial
        dec.set_seed(seed)
        got = dec.speculative_accept(12, draft, dp.reshape(-1), T, top_p)
        rows = np.stack([ref.step(t, 12 + i) for i, t in enumerate(draft)])
        u = [spec_uniform(seed, i) for i in range(K + 1)]
        want = O.speculative_accept(rows, draft, dp, u, T, top_p)
        assert got == want, (trial, got, want)
        outcomes.add(got[0])
        ref.close()
        dec.close()
    print(f"accepted counts seen: {sorted(outcomes)}", flush=True)


def test_speculative_accept_at_cache_end(cuda):
    """Drafts running past max_seq_len: the reference's step_internal gives zero
    logits there (decoder.rs:1066-1089) and acceptance proceeds
    (decoder.rs:588-612), so no error -- the same (accepted, bonus) as the oracle
    over the two verified rows and two zero rows."""
    print("case speculative_accept at the cache end", flush=True)
    V, K, max_seq = 1000, 4, 16
    g = np.random.default_rng(77)
    for trial in range(4):
        ref, dec = make(small(), 4, 4, max_seq=max_seq, seed=60 + trial)
        pre = [int(t) for t in g.integers(0, V, 14)]
        for i, t in enumerate(pre):
            ref.step(t, i)
        dec.prefill_tokens(pre, 0)
        draft = [int(t) for t in g.integers(0, V, K)]
        dp = g.random((K, V)).astype(np.float32) ** 6
        dp /= dp.sum(1, keepdims=True)
        dec.set_seed(5 + trial)
        got = dec.speculative_accept(14, draft, dp.reshape(-1), 1.0, 1.0)
        rows = np.stack([ref.step(t, 14 + i) for i, t in enumerate(draft)])
        assert not rows[2:].any()
        u = [spec_uniform(5 + trial, i) for i in range(K + 1)]
        assert got == O.speculative_accept(rows, draft, dp, u, 1.0, 1.0), trial
        assert dec.kv_len() == max_seq
        ref.close()
        dec.close()


@pytest.mark.parametrize("n,start", [(3, 40), (6, 2400)])
def test_verify_llama_heads_long_prefix(cuda, n, start):
    """head_dim 128, 4 query heads per KV head: 12 and 24 query rows per KV
    head (the 16- and 32-row attention tiles); the 2400-position prefix splits
    the key range 76 ways, more than one pass of the merge."""
    print(f"case verify llama heads n={n} start={start}", flush=True)
    cfg = small(num_layers=1, num_heads=8, num_kv_heads=2, head_dim=128, hidden=1024,
                intermediate=2048, qkv_bias=False)
    max_seq = start + 64
    ref, dec = make(cfg, 4, 4, max_seq=max_seq, seed=43)
    kv = synth.kv_prefill(cfg, 43, start, max_seq)
    for li, (k, v) in enumerate(kv):
        ref.copy_kv(li, k, v, start)
    dec.copy_kv_cache_from_tensors([k for k, _ in kv], [v for _, v in kv], start)
    g = np.random.default_rng(start + n)
    toks = [int(t) for t in g.integers(0, 1000, n)]
    rows = dec.verify_tokens(start, toks)
    want = [ref.step(t, start + i) for i, t in enumerate(toks)]
    err = max(rel(a, b) for a, b in zip(rows, want))
    print(f"verify rows rel err {err:.3g}", flush=True)
    assert len(rows) == n and err < 2e-4
    assert dec.kv_len() == start + n
    ref.close()
    dec.close()

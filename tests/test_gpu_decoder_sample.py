"""Sampled generation on the device against the oracle.

The reference's generate_loop (src/llm/decoder.rs:788-832) pushes each token
onto a 64-token window (859-876), decodes it, applies the repetition penalty
(878-899) and samples (908-1020).  The oracle replays that loop: its decoder
step, its penalty and its sampler with draw u_i = tb_sample_uniform(seed, i),
the library's generator.  The GPU decoder's sampled generate_loop (graph
replays with the sampler tail) must produce the same tokens; so must the
per-token decode_and_sample loop, the EOS path and the steps past the cache.
"""
import numpy as np
import pytest

from oracle import oracle as O
import torchburn_amd as tb
from torchburn_amd import synth
from torchburn_amd.decoder import decoder_from_weights

pytestmark = pytest.mark.gpu

CFG = dict(num_layers=2, hidden=256, intermediate=512, num_heads=4, num_kv_heads=2,
           head_dim=64, vocab=1000, eps=1e-6, rope_theta=1e6, qkv_bias=True)


def make(max_seq, seed=31):
    w = synth.decoder_weights(CFG, seed, 4, 4, 32)
    ocfg = dict(num_layers=2, hidden=256, intermediate=512, num_heads=4, num_kv_heads=2,
                head_dim=64, vocab=1000, group_size=32, max_seq=max_seq, rope_theta=1e6,
                eps=1e-6, wkind=4, lmkind=4)
    return O.Decoder(w, ocfg), decoder_from_weights(w, CFG, group_size=32, max_seq_len=max_seq)


def oracle_generate(ref, first, seq_len, n, T, k, top_p, pen, seed, recent_seed=(), eos=None,
                    window=64):
    recent, toks, nxt, draw = list(recent_seed), [], first, 0
    while len(toks) < n:
        if eos is not None and nxt == eos:
            break
        toks.append(nxt)
        recent.append(nxt)
        recent = recent[-window:]
        lg = ref.step(nxt, seq_len + len(toks) - 1)
        lg = O.repetition_penalty(lg, recent, pen)
        greedy = not np.isfinite(T) or T <= 0 or k == 1
        kk = 1 if greedy else max(1, min(k, lg.size))
        u = tb.sample_uniform(seed, draw)
        nxt, _ = O.sample_logits(lg, T, k, top_p, u)
        if not greedy and kk > 1:
            draw += 1
    return toks


@pytest.mark.parametrize("T,k,top_p,pen", [(0.8, 40, 0.9, 1.1), (1.2, 128, 1.0, 1.0),
                                           (0.0, 40, 1.0, 1.3), (0.7, 2, 0.5, 1.05),
                                           (0.9, 500, 0.95, 1.1), (1.0, 129, 1.0, 1.0),
                                           (0.8, 5000, 0.9, 1.0)])
def test_generate_sampled_matches_oracle(cuda, T, k, top_p, pen):
    print(f"case sampled generate T={T} top_k={k} top_p={top_p} penalty={pen}", flush=True)
    ref, dec = make(128)
    seed = 1234 + k
    seed_ids = list(range(100, 170))      # longer than the window
    want = oracle_generate(ref, 7, 0, 14, T, k, top_p, pen, seed, seed_ids)
    dec.set_seed(seed)
    got, sl = dec.generate_loop(7, 0, 14, temperature=T, top_k=k, top_p=top_p,
                                repetition_penalty=pen, recent_seed=seed_ids)
    assert got == want and sl == 14
    # the same stream through per-token decode_and_sample calls
    dec.reset_kv_cache()
    dec.set_seed(seed)
    recent, toks, nxt = list(seed_ids), [], 7
    for i in range(14):
        toks.append(nxt)
        recent = (recent + [nxt])[-64:]
        nxt = dec.decode_and_sample(nxt, i, T, k, pen, recent, top_p)
    assert toks == want
    ref.close()
    dec.close()


def test_generate_sampled_eos_and_past_cache(cuda):
    ref, dec = make(40)
    seed, T, k, top_p, pen = 99, 0.9, 30, 0.95, 1.2
    full = oracle_generate(ref, 3, 30, 16, T, k, top_p, pen, seed)   # 10 steps in the cache
    ref.close()
    dec.set_seed(seed)
    got, sl = dec.generate_loop(3, 30, 16, temperature=T, top_k=k, top_p=top_p,
                                repetition_penalty=pen)
    assert got == full and sl == 46
    eos = full[5]
    cut = full[:full.index(eos)]
    dec.reset_kv_cache()
    dec.set_seed(seed)
    got, sl = dec.generate_loop(3, 30, 16, temperature=T, top_k=k, top_p=top_p,
                                repetition_penalty=pen, eos_token_id=eos)
    assert got == cut and sl == 30 + len(cut)
    dec.close()


def test_sampler_paths_alternate_in_one_loop(cuda):
    """top_k on either side of the slice path's 128 in one decoder: each path has
    its own sampled-step graph, and switching back and forth keeps the draw
    stream (seeded, the oracle's tokens)."""
    ref, dec = make(128)
    seed = 77
    # each oracle run rewrites positions 0..7 in order before reading them
    want_a = oracle_generate(ref, 11, 0, 8, 0.8, 40, 0.9, 1.1, seed)
    want_b = oracle_generate(ref, 11, 0, 8, 0.8, 300, 0.9, 1.1, seed)
    ref.close()
    for k, want in ((40, want_a), (300, want_b), (40, want_a), (300, want_b)):
        dec.reset_kv_cache()
        dec.set_seed(seed)
        got, _ = dec.generate_loop(11, 0, 8, temperature=0.8, top_k=k, top_p=0.9,
                                   repetition_penalty=1.1)
        assert got == want, k
    dec.close()

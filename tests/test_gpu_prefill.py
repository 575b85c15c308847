"""Parity of the batched prompt prefill with the CPU oracle's step-by-step prefill.

The reference's prefill_tokens (src/llm/decoder.rs:431-447) runs one decoder
step per prompt token and keeps the last step's logits.  The gfx950 decoder
runs prompts of 16 or more in-vocabulary tokens (INT4 projections) as batches:
row RMSNorms, the QKV / O / gate-up / down projections on the FP32-MFMA GEMM,
RoPE + KV append for every row and causal attention over the cache.  The
oracle steps through the same prompt; the prefill's logits, the KV cache it
leaves (through the decode steps that read it) and the greedy continuation
must match.  Metric max|d| / max|ref| (tests/parity/int4.rs:131-141).
"""
import numpy as np
import pytest

from oracle import oracle as O
from torchburn_amd import synth
from torchburn_amd.decoder import decoder_from_weights

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-4


def small(**kw):
    cfg = dict(num_layers=2, hidden=256, intermediate=512, num_heads=4, num_kv_heads=2,
               head_dim=64, vocab=1000, eps=1e-6, rope_theta=1e6, qkv_bias=True)
    cfg.update(kw)
    return cfg


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def run_prefill(cfg, seed, n, start=0, lmkind=4, gs=32, max_seq=512, steps=6):
    print(f"case prefill cfg={cfg} n={n} start={start} lmkind={lmkind} gs={gs}", flush=True)
    w = synth.decoder_weights(cfg, seed, 4, lmkind, gs)
    ocfg = dict(num_layers=cfg["num_layers"], hidden=cfg["hidden"],
                intermediate=cfg["intermediate"], num_heads=cfg["num_heads"],
                num_kv_heads=cfg["num_kv_heads"], head_dim=cfg["head_dim"], vocab=cfg["vocab"],
                group_size=gs, max_seq=max_seq, rope_theta=cfg["rope_theta"], eps=cfg["eps"],
                wkind=4, lmkind=lmkind)
    ref = O.Decoder(w, ocfg)
    dec = decoder_from_weights(w, cfg, group_size=gs, max_seq_len=max_seq)
    if start:
        kv = synth.kv_prefill(cfg, seed, start, max_seq)
        for li, (k, v) in enumerate(kv):
            ref.copy_kv(li, k, v, start)
        dec.copy_kv_cache_from_tensors([k for k, _ in kv], [v for _, v in kv], start)
    g = np.random.default_rng(seed)
    prompt = [int(t) for t in g.integers(0, cfg["vocab"], n)]
    for i, t in enumerate(prompt):
        lo = ref.step(t, start + i)
    assert dec.prefill_tokens(prompt, start) == start + n
    assert dec.kv_len() == start + n
    err = rel(dec.get_logits(), lo)
    print(f"prefill logits rel err {err:.3g}", flush=True)
    assert err < LOGIT_TOL
    # Decode steps over the cache the prefill wrote.
    tok, worst = O.argmax(lo), 0.0
    for i in range(steps):
        lo = ref.step(tok, start + n + i)
        lg, am = dec._step(tok, start + n + i, True)
        worst = max(worst, rel(lg, lo))
        nxt = O.argmax(lo)
        assert am == nxt, f"step {i}: GPU argmax {am} != oracle {nxt}"
        tok = nxt
    print(f"decode-after-prefill logits rel err {worst:.3g}", flush=True)
    assert worst < LOGIT_TOL
    ref.close()
    dec.close()


def test_prefill_small(cuda):
    run_prefill(small(), 21, 37)


def test_prefill_chunks_after_cached_prefix(cuda):
    """A 300-token prompt after 20 cached positions: two 256-row chunks, the
    second attending over the first chunk's KV rows."""
    run_prefill(small(), 22, 300, start=20, max_seq=400)


def test_prefill_llama_head_layout_fp32_lm_head(cuda):
    cfg = small(num_heads=8, num_kv_heads=2, head_dim=128, hidden=1024, intermediate=2048,
                qkv_bias=False)
    run_prefill(cfg, 23, 70, start=5, lmkind=32)


def test_prefill_threshold_g64_int8_lm_head(cuda):
    run_prefill(small(), 24, 16, gs=64, lmkind=8)


def test_prefill_group64_v2_blocks(cuda):
    """Group 64, vocab 1024: the batched projections read v2 blocks for QKV, O
    and down and the lm_head (MFMA V2 path)."""
    run_prefill(small(vocab=1024), 28, 100, start=7, gs=64)


def test_prefill_qwen_layer_shape(cuda):
    cfg = small(num_layers=1, hidden=896, intermediate=4864, num_heads=14, num_kv_heads=2)
    run_prefill(cfg, 25, 260, max_seq=300)


@pytest.mark.parametrize("heads", [(4, 4), (16, 1)])
def test_prefill_mha_and_wide_groups(cuda, heads):
    cfg = small(num_layers=1, num_heads=heads[0], num_kv_heads=heads[1],
                hidden=64 * heads[0] if heads[0] > 4 else 256)
    run_prefill(cfg, 26, 65, start=3)


def test_prefill_short_prompt_uses_steps(cuda):
    run_prefill(small(), 27, 15)

"""The device quantizers and the quantized-checkpoint path against the CPU oracle.

  quantize_weight_int4_grouped   bit-exact against the oracle's restatement of
      python/torchburn/quantization.py:53-118 (pinned there against a numpy
      closed form): ties, zero groups, K % 64 != 0 at group 32, host input,
      group sizes other than 32 / 64 (1, 3, 100, 128, 512), odd K refused
  quantize_weight_int8           bit-exact against fused_ops.rs:554-589's restatement
  unpack v2 -> v1                the loader's migration (loader.py:539-561): nibbles
      unchanged, scales = binary16 rounding of the originals
  QuantizedLinear                forward against the oracle GEMV (1e-4)
  checkpoint                     a small Hugging Face-layout checkpoint quantized on
      the GPU equals the oracle quantizer's tensors bit for bit; the cache round
      trip and the v2 cache reproduce them; the decoder built from them matches
      the oracle decoder (2e-4, identical greedy tokens)
"""
import json

import numpy as np
import pytest
import torch

from oracle import oracle as O
import torchburn_amd as tb
from torchburn_amd import checkpoint as ck

pytestmark = pytest.mark.gpu


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("n,k,gs", [(37, 896, 64), (64, 4096, 32), (5, 96, 32), (3, 64, 64),
                                    (7, 768, 128), (6, 200, 100), (4, 96, 3), (3, 1536, 512),
                                    (5, 10, 1)])
def test_quantize_int4_bit_exact(cuda, n, k, gs):
    print(f"case quantize_weight_int4_grouped n={n} k={k} gs={gs}", flush=True)
    g = np.random.default_rng(n * k + gs)
    w = g.standard_normal((n, k)).astype(np.float32)
    w[0, :gs] = 0.0                                    # zero group -> scale 1e-8
    s0 = np.abs(w[1, :gs]).max() / np.float32(7.0)
    w[1, min(3, gs - 1)] = np.float32(2.5) * s0        # an exact tie (if representable)
    w[2, :gs] *= np.float32(1e-12)                     # tiny group: scale clamps at 1e-8
    wq_ref, s_ref = O.quantize_int4_grouped(w, gs)
    wq, s = tb.quantize_weight_int4_grouped(torch.from_numpy(w).to(cuda), group_size=gs)
    assert np.array_equal(wq.cpu().numpy(), wq_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)
    # host input, chunked rows; the result stays on the host
    wq2, s2 = tb.quantize_weight_int4_grouped(torch.from_numpy(w), group_size=gs, chunk_size=2)
    assert wq2.device.type == "cpu" and np.array_equal(wq2.numpy(), wq_ref)
    assert np.array_equal(s2.numpy(), s_ref)


def test_quantize_int4_errors(cuda):
    w = torch.zeros((4, 96), device=cuda)
    with pytest.raises(ValueError, match="divisible"):
        tb.quantize_weight_int4_grouped(w, group_size=64)
    with pytest.raises(RuntimeError, match="odd"):
        tb.quantize_weight_int4_grouped(torch.zeros((4, 9), device=cuda), group_size=3)


def test_quantize_int8_bit_exact(cuda):
    print("case quantize_weight_int8", flush=True)
    g = np.random.default_rng(7)
    w = g.standard_normal((50, 1000)).astype(np.float32)
    w[1] = 0.0
    w[2] = np.float32(4e-9)
    w[3, :3] = [127.0, 2.5, -2.5]
    w[3, 3:] = 0.0
    q_ref, s_ref = O.quantize_int8(w)
    q, s = tb.quantize_weight_int8(torch.from_numpy(w).to(cuda))
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(s.cpu().numpy(), s_ref)
    assert list(q[3, :3].cpu().numpy()) == [127, 3, -3]


def test_unpack_v2_to_v1(cuda):
    g = np.random.default_rng(8)
    wq, sc = O.quantize_int4_grouped(g.standard_normal((33, 576)).astype(np.float32), 64)
    blocked = O.pack_v1_to_v2(wq, sc, 576)
    w1, s1 = tb.unpack_rows_w4a32_group64_v2_to_v1(torch.from_numpy(blocked).to(cuda))
    assert np.array_equal(w1.cpu().numpy(), wq)
    assert np.array_equal(s1.cpu().numpy(), sc.astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("bits", [4, 8])
def test_quantized_linear_forward(cuda, bits):
    g = np.random.default_rng(9)
    lin = torch.nn.Linear(512, 300, bias=True)
    ql = tb.QuantizedLinear.from_float(lin, bits=bits, group_size=64)
    x = g.standard_normal((3, 512)).astype(np.float32)
    y = ql(torch.from_numpy(x).to(cuda)).cpu().numpy()
    w = lin.weight.detach().numpy().astype(np.float32)
    b = lin.bias.detach().numpy().astype(np.float32)
    if bits == 4:
        wq, sc = O.quantize_int4_grouped(w, 64)
        ref = O.gemm_w4(x, wq, sc, b, group_size=64)
    else:
        q, s = O.quantize_int8(w)
        ref = O.gemv_w8(x, q, s, b)
    assert rel(y, ref) < 1e-4


# ---------------------------------------------------------------- checkpoint ---

def make_checkpoint(path, tied, bias, vocab, seed):
    """A 2-layer Hugging Face-layout checkpoint (two shards) with config.json."""
    from safetensors.torch import save_file
    H, I, hq, hkv, hd = 128, 256, 2, 1, 64
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, sd=0.05: torch.randn(*s, generator=g) * sd
    t = {"model.embed_tokens.weight": r(vocab, H, sd=0.5), "model.norm.weight": 1 + r(H)}
    for i in range(2):
        p = f"model.layers.{i}."
        t[p + "input_layernorm.weight"] = 1 + r(H, sd=0.1)
        t[p + "post_attention_layernorm.weight"] = 1 + r(H, sd=0.1)
        for nm, rows in (("q_proj", hq * hd), ("k_proj", hkv * hd), ("v_proj", hkv * hd)):
            t[p + f"self_attn.{nm}.weight"] = r(rows, H)
            if bias:
                t[p + f"self_attn.{nm}.bias"] = r(rows, sd=0.02)
        t[p + "self_attn.o_proj.weight"] = r(H, hq * hd)
        t[p + "mlp.gate_proj.weight"] = r(I, H)
        t[p + "mlp.up_proj.weight"] = r(I, H)
        t[p + "mlp.down_proj.weight"] = r(H, I)
    if not tied:
        t["lm_head.weight"] = r(vocab, H)
    keys = sorted(t)
    save_file({k: t[k].contiguous() for k in keys[: len(keys) // 2]},
              str(path / "model-00001-of-00002.safetensors"))
    save_file({k: t[k].contiguous() for k in keys[len(keys) // 2:]},
              str(path / "model-00002-of-00002.safetensors"))
    cfg = dict(architectures=["Qwen2ForCausalLM" if bias else "LlamaForCausalLM"],
               model_type="qwen2" if bias else "llama", hidden_size=H, intermediate_size=I,
               num_hidden_layers=2, num_attention_heads=hq, num_key_value_heads=hkv,
               vocab_size=vocab, rms_norm_eps=1e-6, rope_theta=1e6,
               tie_word_embeddings=tied, attention_bias=bias)
    (path / "config.json").write_text(json.dumps(cfg))
    return {k: v.numpy() for k, v in t.items()}, cfg


def oracle_weights(t, cfg, tied):
    """The oracle decoder's weight dict from the float tensors, quantized by the
    oracle's restatement of the reference quantizer (group 64)."""
    q = lambda w: O.quantize_int4_grouped(np.ascontiguousarray(w, np.float32), 64)
    layers = []
    for i in range(2):
        p = f"model.layers.{i}."
        qkv = np.concatenate([t[p + f"self_attn.{n}.weight"] for n in ("q_proj", "k_proj",
                                                                       "v_proj")], 0)
        lw = dict(in_norm=t[p + "input_layernorm.weight"],
                  post_norm=t[p + "post_attention_layernorm.weight"])
        lw["qkv_w"], lw["qkv_s"] = q(qkv)
        lw["o_w"], lw["o_s"] = q(t[p + "self_attn.o_proj.weight"])
        for nm, key in (("gate", "gate_proj"), ("up", "up_proj"), ("down", "down_proj")):
            lw[nm + "_w"], lw[nm + "_s"] = q(t[p + f"mlp.{key}.weight"])
        if cfg["attention_bias"]:
            lw["qkv_b"] = np.concatenate([t[p + f"self_attn.{n}.bias"]
                                          for n in ("q_proj", "k_proj", "v_proj")], 0)
        layers.append(lw)
    lm_w, lm_s = q(t["model.embed_tokens.weight"] if tied else t["lm_head.weight"])
    return dict(embed=t["model.embed_tokens.weight"], final_norm=t["model.norm.weight"],
                lm_head_w=lm_w, lm_head_s=lm_s, layers=layers)


@pytest.mark.parametrize("tied,bias,vocab", [(True, True, 320), (False, False, 300)])
def test_checkpoint_quantize_cache_and_decode(cuda, tmp_path, monkeypatch, tied, bias, vocab):
    print(f"case checkpoint tied={tied} bias={bias} vocab={vocab}", flush=True)
    monkeypatch.setattr(ck, "CACHE_DIR", str(tmp_path / "home"))
    t, cfg = make_checkpoint(tmp_path, tied, bias, vocab, seed=vocab)
    sd, dcfg, path = ck.load_quantized(str(tmp_path), "int4")
    assert path == str(tmp_path / "torchburn_int4_g64.safetensors")
    ow = oracle_weights(t, cfg, tied)
    for i, lw in enumerate(ow["layers"]):
        p = f"layers.{i}."
        assert np.array_equal(sd[p + "self_attn.qkv_proj.qweight"].cpu().numpy(), lw["qkv_w"])
        assert np.array_equal(sd[p + "self_attn.qkv_proj.scales"].cpu().numpy(), lw["qkv_s"])
        assert np.array_equal(sd[p + "mlp.down_proj.qweight"].cpu().numpy(), lw["down_w"])
        assert (p + "self_attn.qkv_proj.bias" in sd) == bias
    assert np.array_equal(sd["lm_head.qweight"].cpu().numpy(), ow["lm_head_w"])
    # cache hit: the same tensors, read from the file
    sd2, _, path2 = ck.load_quantized(str(tmp_path), "int4")
    assert path2 == path and sd2.keys() == sd.keys()
    assert all(torch.equal(sd[k], sd2[k]) for k in sd)
    # decoder from the cache tensors vs the oracle decoder
    max_seq = 64
    ocfg = dict(num_layers=2, hidden=128, intermediate=256, num_heads=2, num_kv_heads=1,
                head_dim=64, vocab=vocab, group_size=64, max_seq=max_seq, rope_theta=1e6,
                eps=1e-6, wkind=4, lmkind=4)
    ref = O.Decoder(ow, ocfg)
    dec = ck.decoder_from_state_dict(sd2, dcfg, max_seq_len=max_seq)
    tok, worst = 5, 0.0
    for step in range(6):
        lo = ref.step(tok, step)
        lg, am = dec._step(tok, step, True)
        worst = max(worst, rel(lg, lo))
        assert am == O.argmax(lo)
        tok = am
    print(f"checkpoint decoder rel err {worst:.3g}", flush=True)
    assert worst < 2e-4
    dec.close()
    ref.close()
    # v2 cache: preferred by the search, migrated back to v1 tensors with
    # binary16 scales
    v2 = ck.migrate_cache_to_v2(str(tmp_path))
    assert ck.find_cache(str(tmp_path)) == v2
    sd3, _, path3 = ck.load_quantized(str(tmp_path), "int4")
    assert path3 == v2
    for k in sd:
        if k.endswith(".qweight"):
            assert torch.equal(sd3[k], sd[k])
        elif k.endswith(".scales"):
            assert torch.equal(sd3[k], sd[k].half().float())
    # The v2 cache carries binary16 scales for every projection (gate / up too):
    # the decoder over it matches the oracle decoder over those scales.
    r16 = lambda a: a.astype(np.float16).astype(np.float32)
    ow16 = dict(ow, lm_head_s=r16(ow["lm_head_s"]),
                layers=[{k: (r16(v) if k.endswith("_s") else v) for k, v in lw.items()}
                        for lw in ow["layers"]])
    ref2 = O.Decoder(ow16, ocfg)
    d2 = ck.decoder_from_state_dict(sd3, dcfg, max_seq_len=max_seq)
    for j, t_ in enumerate((3, 9, 17)):
        lo = ref2.step(t_, j)
        lg, am = d2._step(t_, j, True)
        assert rel(lg, lo) < 2e-4 and am == O.argmax(lo)
    d2.close()
    ref2.close()

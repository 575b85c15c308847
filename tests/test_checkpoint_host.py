"""Host logic of the checkpoint loader (torchburn_amd/checkpoint.py), no GPU:
the config fields and refusals (python/torchburn/llm/config.py:44-174), the
tensor-name candidates (python/torchburn/llm/loader.py:208-363) and the cache
search order (loader.py:86-110)."""
import os

import pytest

from torchburn_amd import checkpoint as ck
from torchburn_amd import UnsupportedOpError


def test_config_defaults_and_families():
    c = ck.decoder_config({"hidden_size": 64, "num_attention_heads": 4, "model_type": "qwen2"})
    assert c["head_dim"] == 16 and c["num_key_value_heads"] == 4
    assert c["qkv_bias"] and c["tie_word_embeddings"]          # Qwen defaults
    assert c["rope_theta"] == 10000.0 and c["vocab_size"] == 151936
    assert c["intermediate_size"] == 256 and c["rms_norm_eps"] == 1e-6
    l = ck.decoder_config({"hidden_size": 4096, "num_attention_heads": 32,
                           "num_key_value_heads": 8, "model_type": "llama",
                           "rope_parameters": {"rope_theta": 500000.0},
                           "head_dim": None, "rms_norm_eps": 1e-5})
    assert l["head_dim"] == 128 and l["num_key_value_heads"] == 8
    assert not l["qkv_bias"] and not l["tie_word_embeddings"] and l["rope_theta"] == 5e5
    assert ck.decoder_config({"model_type": "llama", "attention_bias": True})["qkv_bias"]


@pytest.mark.parametrize("cfg", [{"model_type": "mixtral", "num_local_experts": 8},
                                 {"model_type": "gemma"}, {"model_type": "gpt2"},
                                 {"model_type": "llama", "hidden_act": "gelu"},
                                 {"model_type": "qwen3", "qk_layernorm": True}])
def test_config_refuses_other_families(cfg):
    with pytest.raises(UnsupportedOpError):
        ck.decoder_config(cfg)


def test_candidate_names():
    assert ck.candidate_names("q_proj", 3)[:2] == ["layers.3.self_attn.q_proj.weight",
                                                   "model.layers.3.self_attn.q_proj.weight"]
    assert ck.candidate_names("down_proj", 0, "bias")[1] == "model.layers.0.mlp.down_proj.bias"
    assert "model.layers.2.mlp.w1.weight" in ck.candidate_names("gate_proj", 2)
    assert ck.candidate_names("input_layernorm", 1)[1] == "model.layers.1.input_layernorm.weight"
    assert "model.embed_tokens.weight" in ck.candidate_names("embed_tokens")
    assert "transformer.ln_f.weight" in ck.candidate_names("norm")


def test_cache_search_order(tmp_path, monkeypatch):
    d = tmp_path / "m"
    d.mkdir()
    (d / "config.json").write_text("{}")
    (d / "model.safetensors").write_bytes(b"")
    home = tmp_path / "home"
    monkeypatch.setattr(ck, "CACHE_DIR", str(home))
    assert ck.find_cache(str(d)) is None
    home.mkdir()
    (home / "m_torchburn_int4_g64.safetensors").write_bytes(b"")
    assert ck.find_cache(str(d)).endswith("home/m_torchburn_int4_g64.safetensors")
    (d / "torchburn_int4_g64.safetensors").write_bytes(b"")
    assert ck.find_cache(str(d)) == str(d / "torchburn_int4_g64.safetensors")
    (home / "m_torchburn_int4_g64_v2.safetensors").write_bytes(b"")
    assert ck.find_cache(str(d)).endswith("m_torchburn_int4_g64_v2.safetensors")
    files, cfg = ck.checkpoint_files(str(d))
    assert files == [str(d / "model.safetensors")] and cfg.endswith("config.json")
    assert ck.cache_names("int8")[1] == "torchburn_int8_g64.safetensors"

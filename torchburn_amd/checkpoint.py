"""Quantized checkpoints for the decoder, on the device.

Mirrors the reference loader's quantized path (python/torchburn/llm/loader.py:
``load`` 61-181, ``_stream_quantize_safetensors`` 183-537, ``_migrate_v2_state_dict``
539-561, ``migrate_cache_to_v2`` 563-608) and the part of ``ModelConfig.from_dict``
(python/torchburn/llm/config.py:44-174) that the decoder needs:

* a Hugging Face safetensors checkpoint is quantized layer by layer on the GPU
  (``tb_quantize_weight_int4_grouped`` / ``tb_quantize_weight_int8``), Q/K/V fused
  into one projection, and written as the reference's disk cache
  ``torchburn_{quant}_g64.safetensors`` with its state-dict keys
  (``layers.{i}.self_attn.qkv_proj.qweight`` / ``.scales`` / ``.bias`` ...);
* a cache file is read straight into device memory; a v2 cache
  (``torchburn_int4_g64_v2.safetensors``: 34-byte blocks, no ``.scales``) is
  migrated to v1 tensors by ``tb_unpack_rows_w4a32_group64_v2_to_v1``;
* ``create_decoder_from_checkpoint`` builds a ``RustQwenDecoder`` from it.

Only local files are read (there is no download).  The decoder runs the dense
pre-norm RoPE / SwiGLU families (Llama, Qwen2, Mistral); configurations with
experts, learned positions, per-head Q/K norms, parallel residuals, offset norms
or a non-SiLU activation are refused with UnsupportedOpError.
"""
from __future__ import annotations

import json
import os
from pathlib import Path
from typing import Dict, List, Optional, Tuple

import torch

from . import _lib
from ._lib import UnsupportedOpError
from .quantization import (pack_rows_w4a32_group64_v1_to_v2, quantize_weight_int4_grouped,
                           quantize_weight_int8, unpack_rows_w4a32_group64_v2_to_v1)

CACHE_DIR = os.path.expanduser("~/.cache/torchburn")


# ---------------------------------------------------------------------------
# Configuration (config.py:44-174, the fields the decoder reads)
# ---------------------------------------------------------------------------

def decoder_config(data: Dict) -> Dict:
    """Decoder configuration from a Hugging Face config.json dict, with the
    reference's defaults for absent keys (config.py:10-41, 44-174)."""
    hidden = int(data.get("hidden_size", 896))
    heads = int(data.get("num_attention_heads", 14))
    head_dim = int(data.get("head_dim", hidden // max(heads, 1)) or hidden // max(heads, 1))
    theta = data.get("rope_theta")
    if theta is None and "rope_parameters" in data:
        theta = data["rope_parameters"].get("rope_theta")
    if theta is None:
        theta = 10000.0
    arch = (data.get("architectures") or [""])[0].lower()
    model_type = str(data.get("model_type", "")).lower()
    is_qwen = "qwen" in arch or "qwen" in model_type
    is_gemma = "gemma" in arch or "gemma" in model_type
    unsupported = []
    if data.get("num_experts") or data.get("n_routed_experts") or data.get("num_local_experts"):
        unsupported.append("mixture-of-experts layers")
    if is_gemma or data.get("norm_type", "standard") != "standard":
        unsupported.append("offset RMSNorm / scaled embeddings")
    if "gpt2" in arch or "gpt2" in model_type or "neox" in arch or "neox" in model_type:
        unsupported.append("learned positions / parallel residual")
    if data.get("use_parallel_residual") or data.get("qk_layernorm"):
        unsupported.append("parallel residual or per-head Q/K norm")
    act = str(data.get("hidden_act", "silu")).lower()
    if act not in ("silu", "swish"):
        unsupported.append(f"activation {act}")
    if unsupported:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} the decoder runs dense pre-norm RoPE / SwiGLU models; "
            f"this checkpoint has {', '.join(unsupported)}")
    return dict(
        vocab_size=int(data.get("vocab_size", 151936)),
        hidden_size=hidden,
        intermediate_size=int(data.get("intermediate_size", hidden * 4)),
        num_hidden_layers=int(data.get("num_hidden_layers", 24)),
        num_attention_heads=heads,
        num_key_value_heads=int(data.get("num_key_value_heads", data.get("num_kv_heads", heads))),
        head_dim=head_dim,
        rms_norm_eps=float(data.get("rms_norm_eps", 1e-6)),
        rope_theta=float(theta),
        qkv_bias=bool(data.get("qkv_bias", data.get("attention_bias", is_qwen))),
        tie_word_embeddings=bool(data.get("tie_word_embeddings", is_qwen)),
    )


# ---------------------------------------------------------------------------
# Tensor names of the checkpoint (loader.py:208-363, dense families)
# ---------------------------------------------------------------------------

_LAYER_ALIASES = {
    "input_layernorm": ["model.layers.{i}.input_layernorm.weight",
                        "transformer.h.{i}.ln_1.weight",
                        "transformer.layers.{i}.input_layernorm.weight",
                        "layers.{i}.operator_norm.weight"],
    "post_attention_layernorm": ["model.layers.{i}.post_attention_layernorm.weight",
                                 "transformer.h.{i}.ln_2.weight",
                                 "transformer.layers.{i}.post_attention_layernorm.weight"],
    "q_proj": ["model.layers.{i}.self_attn.q_proj.{p}", "transformer.h.{i}.attn.q_proj.{p}",
               "transformer.layers.{i}.self_attn.q_proj.{p}"],
    "k_proj": ["model.layers.{i}.self_attn.k_proj.{p}", "transformer.h.{i}.attn.k_proj.{p}",
               "transformer.layers.{i}.self_attn.k_proj.{p}"],
    "v_proj": ["model.layers.{i}.self_attn.v_proj.{p}", "transformer.h.{i}.attn.v_proj.{p}",
               "transformer.layers.{i}.self_attn.v_proj.{p}"],
    "o_proj": ["model.layers.{i}.self_attn.o_proj.{p}", "transformer.h.{i}.attn.out_proj.{p}",
               "transformer.layers.{i}.self_attn.o_proj.{p}",
               "model.layers.{i}.self_attn.dense.{p}"],
    "gate_proj": ["model.layers.{i}.mlp.gate_proj.{p}", "transformer.h.{i}.mlp.gate_proj.{p}",
                  "transformer.layers.{i}.mlp.gate_proj.{p}", "model.layers.{i}.mlp.w1.{p}"],
    "up_proj": ["model.layers.{i}.mlp.up_proj.{p}", "transformer.h.{i}.mlp.up_proj.{p}",
                "transformer.layers.{i}.mlp.up_proj.{p}", "model.layers.{i}.mlp.w3.{p}"],
    "down_proj": ["model.layers.{i}.mlp.down_proj.{p}", "transformer.h.{i}.mlp.down_proj.{p}",
                  "transformer.layers.{i}.mlp.down_proj.{p}", "model.layers.{i}.mlp.w2.{p}"],
}
_GLOBAL_ALIASES = {
    "embed_tokens": ["transformer.wte.weight",
                     "transformer.embedding.word_embeddings.weight", "word_embeddings.weight",
                     "embeddings.word_embeddings.weight"],
    "norm": ["model.norm.weight", "transformer.ln_f.weight", "transformer.norm.weight",
             "model.final_layernorm.weight"],
    "lm_head": ["lm_head.weight", "model.lm_head.weight"],
}


def candidate_names(key: str, layer: Optional[int] = None, part: str = "weight") -> List[str]:
    """The checkpoint names tried for a tensor, in order (loader.py:208-363)."""
    if layer is None:
        return [key, f"model.{key}", f"{key}.weight", f"model.{key}.weight",
                *_GLOBAL_ALIASES.get(key, [])]
    if key.endswith("layernorm"):
        base = f"layers.{layer}.{key}.weight"
    else:
        owner = "mlp" if key in ("gate_proj", "up_proj", "down_proj") else "self_attn"
        base = f"layers.{layer}.{owner}.{key}.{part}"
    names = [base, f"model.{base}"]
    names += [n.format(i=layer, p=part) for n in _LAYER_ALIASES[key] if n.format(i=layer, p=part)
              not in names]
    return names


class _Checkpoint:
    """Name -> file index over safetensors shards; tensors are read one at a time."""

    def __init__(self, files: List[str]):
        from safetensors import safe_open
        self._safe_open = safe_open
        self.index: Dict[str, str] = {}
        for f in files:
            with safe_open(f, framework="pt", device="cpu") as sf:
                for k in sf.keys():
                    self.index[k] = f

    def get(self, names: List[str]) -> Optional[torch.Tensor]:
        for n in names:
            if n in self.index:
                with self._safe_open(self.index[n], framework="pt", device="cpu") as sf:
                    return sf.get_tensor(n)
        return None

    def require(self, names: List[str]) -> torch.Tensor:
        t = self.get(names)
        if t is None:
            raise KeyError(f"Required tensor '{names[0]}' is missing from the checkpoint; the "
                           "model architecture is not compatible with TorchBurn's decoder")
        return t


def checkpoint_files(model_dir: str) -> Tuple[List[str], str]:
    """(sorted *.safetensors shards, config.json) of a local model directory
    (loader.py:610-642, local case).  Cache files are not shards."""
    cfg = os.path.join(model_dir, "config.json")
    if not os.path.isfile(cfg):
        raise FileNotFoundError(f"no config.json in {model_dir}")
    files = sorted(os.path.join(model_dir, f) for f in os.listdir(model_dir)
                   if f.endswith(".safetensors") and not f.startswith("torchburn_"))
    if not files:
        raise FileNotFoundError(f"no .safetensors weights in {model_dir}")
    return files, cfg


# ---------------------------------------------------------------------------
# Streaming quantization (loader.py:183-537)
# ---------------------------------------------------------------------------

def _quant(w: torch.Tensor, quant: str, group_size: int, dev: torch.device):
    w = w.to(dev, torch.float32)
    if quant == "int4":
        return quantize_weight_int4_grouped(w, group_size=group_size)
    return quantize_weight_int8(w)


def quantize_checkpoint(model_dir: str, quant: str = "int4", group_size: int = 64,
                        device: Optional[torch.device] = None,
                        save_cache_path: Optional[str] = None) -> Tuple[Dict, Dict]:
    """Quantizes a local safetensors checkpoint layer by layer on the GPU.

    Returns (state dict on the device with the reference's cache keys, decoder
    config).  Q, K and V are concatenated into one projection before
    quantization; a tied lm_head is quantized from the embedding.  With
    ``save_cache_path`` the state dict is written there as safetensors."""
    if quant not in ("int4", "int8"):
        raise ValueError(f"quant must be 'int4' or 'int8', got {quant!r}")
    dev = device or torch.device("cuda", torch.cuda.current_device())
    files, cfg_path = checkpoint_files(model_dir)
    with open(cfg_path, "r", encoding="utf-8") as f:
        cfg = decoder_config(json.load(f))
    ck = _Checkpoint(files)
    sd: Dict[str, torch.Tensor] = {}
    emb = ck.require(candidate_names("embed_tokens")).to(dev, torch.float32)
    sd["embed_tokens.weight"] = emb
    sd["norm.weight"] = ck.require(candidate_names("norm")).to(dev, torch.float32)
    for i in range(cfg["num_hidden_layers"]):
        p = f"layers.{i}."
        sd[p + "input_layernorm.weight"] = \
            ck.require(candidate_names("input_layernorm", i)).to(dev, torch.float32)
        # an absent post-attention norm keeps RMSNorm's initial weight of ones
        post = ck.get(candidate_names("post_attention_layernorm", i))
        sd[p + "post_attention_layernorm.weight"] = (
            post.to(dev, torch.float32) if post is not None
            else torch.ones(cfg["hidden_size"], dtype=torch.float32, device=dev))
        qkv = torch.cat([ck.require(candidate_names(n, i)).to(dev, torch.float32)
                         for n in ("q_proj", "k_proj", "v_proj")], 0)
        sd[p + "self_attn.qkv_proj.qweight"], sd[p + "self_attn.qkv_proj.scales"] = \
            _quant(qkv, quant, group_size, dev)
        del qkv
        if cfg["qkv_bias"]:
            bs = [ck.get(candidate_names(n, i, "bias")) for n in ("q_proj", "k_proj", "v_proj")]
            if all(b is not None for b in bs):
                sd[p + "self_attn.qkv_proj.bias"] = torch.cat(
                    [b.to(dev, torch.float32) for b in bs], 0)
        for mod, names in (("self_attn.o_proj", "o_proj"), ("mlp.gate_proj", "gate_proj"),
                           ("mlp.up_proj", "up_proj"), ("mlp.down_proj", "down_proj")):
            qw, qs = _quant(ck.require(candidate_names(names, i)), quant, group_size, dev)
            sd[p + mod + ".qweight"], sd[p + mod + ".scales"] = qw, qs
    lm = emb if cfg["tie_word_embeddings"] else ck.require(candidate_names("lm_head"))
    sd["lm_head.qweight"], sd["lm_head.scales"] = _quant(lm, quant, group_size, dev)
    if save_cache_path:
        save_quantized_cache(sd, save_cache_path)
    return sd, cfg


# ---------------------------------------------------------------------------
# The disk cache (loader.py:86-181, 523-537, 539-608)
# ---------------------------------------------------------------------------

def cache_names(quant: str) -> List[str]:
    """Cache file names in the order the reference tries them (loader.py:88-96)."""
    return [f"torchburn_{quant}_g64_v2.safetensors", f"torchburn_{quant}_g64.safetensors",
            f"torchburn_{quant}_g64.pt"]


def find_cache(model_dir: str, quant: str = "int4") -> Optional[str]:
    """The first existing cache: each name beside the model, then under
    ~/.cache/torchburn as {dirname}_{name} (loader.py:97-110)."""
    for name in cache_names(quant):
        for cand in (os.path.join(model_dir, name),
                     os.path.join(CACHE_DIR, f"{Path(model_dir).name}_{name}")):
            if os.path.isfile(cand):
                return cand
    return None


def save_quantized_cache(sd: Dict[str, torch.Tensor], path: str) -> None:
    """Writes the state dict as safetensors (contiguous host copies)."""
    import safetensors.torch
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    safetensors.torch.save_file({k: v.detach().contiguous().cpu() for k, v in sd.items()}, path)


def migrate_v2_state_dict(sd: Dict[str, torch.Tensor]) -> Dict[str, torch.Tensor]:
    """v2 ``.qweight`` blocks -> v1 ``.qweight`` + ``.scales`` (loader.py:539-561),
    on the device."""
    out = {}
    for key, t in sd.items():
        if key.endswith(".qweight") and t.ndim == 2 and t.dtype == torch.uint8 \
                and t.shape[1] % 34 == 0 and key.replace(".qweight", ".scales") not in sd:
            out[key], out[key.replace(".qweight", ".scales")] = \
                unpack_rows_w4a32_group64_v2_to_v1(t)
        else:
            out[key] = t
    return out


def load_quantized_cache(path: str, device: Optional[torch.device] = None) -> Dict:
    """A cache file read into device memory; a v2 file is migrated to v1 tensors.
    Loaders that execute nothing from the file only: safetensors, or torch.load
    with weights_only=True for the .pt form."""
    dev = device or torch.device("cuda", torch.cuda.current_device())
    if path.endswith(".safetensors"):
        import safetensors.torch
        sd = safetensors.torch.load_file(path, device=str(dev))
    else:
        sd = {k: v.to(dev) for k, v in torch.load(path, map_location="cpu",
                                                   weights_only=True).items()}
    if os.path.basename(path).endswith("_v2.safetensors"):
        sd = migrate_v2_state_dict(sd)
    return sd


def migrate_cache_to_v2(model_dir: str, quant: str = "int4") -> str:
    """Writes torchburn_int4_g64_v2.safetensors beside a v1 cache (loader.py:563-608):
    every INT4 projection re-packed as 34-byte blocks (the v1 nibbles re-quantize
    to themselves; the scales become binary16)."""
    src = os.path.join(model_dir, f"torchburn_{quant}_g64.safetensors")
    if not os.path.isfile(src):
        src = os.path.join(CACHE_DIR, f"{Path(model_dir).name}_torchburn_{quant}_g64.safetensors")
    sd = load_quantized_cache(src)
    out = {}
    for key, t in sd.items():
        skey = key.replace(".qweight", ".scales")
        if key.endswith(".qweight") and skey in sd and t.dtype == torch.uint8:
            out[key] = pack_rows_w4a32_group64_v1_to_v2(t, sd[skey], t.shape[1] * 2)
        elif key.endswith(".scales") and key.replace(".scales", ".qweight") in sd \
                and sd[key.replace(".scales", ".qweight")].dtype == torch.uint8:
            continue
        else:
            out[key] = t
    dst = os.path.join(model_dir, f"torchburn_{quant}_g64_v2.safetensors")
    save_quantized_cache(out, dst)
    return dst


def load_quantized(model_dir: str, quant: str = "int4", device: Optional[torch.device] = None,
                   group_size: int = 64) -> Tuple[Dict, Dict, str]:
    """(state dict on the device, decoder config, cache path): the cache when
    one exists, else a streaming quantization that writes it beside the model
    (or under ~/.cache/torchburn when the directory is read-only)
    (loader.py:86-181)."""
    with open(checkpoint_files(model_dir)[1], "r", encoding="utf-8") as f:
        cfg = decoder_config(json.load(f))
    hit = find_cache(model_dir, quant)
    if hit:
        return load_quantized_cache(hit, device), cfg, hit
    path = os.path.join(model_dir, f"torchburn_{quant}_g64.safetensors")
    try:
        probe = path + ".tmp"
        with open(probe, "w") as f:
            f.write("ok")
        os.remove(probe)
    except OSError:
        path = os.path.join(CACHE_DIR, f"{Path(model_dir).name}_torchburn_{quant}_g64.safetensors")
    sd, cfg = quantize_checkpoint(model_dir, quant, group_size, device, save_cache_path=path)
    return sd, cfg, path


def decoder_from_state_dict(sd: Dict, cfg: Dict, max_seq_len: int = 4096,
                            group_size: int = 64):
    """RustQwenDecoder over a quantized state dict with the cache's keys."""
    from .decoder import RustQwenDecoder
    layers = []
    for i in range(cfg["num_hidden_layers"]):
        p = f"layers.{i}."
        caps = [sd[p + "input_layernorm.weight"],
                sd[p + "self_attn.qkv_proj.qweight"], sd[p + "self_attn.qkv_proj.scales"],
                sd[p + "self_attn.o_proj.qweight"], sd[p + "self_attn.o_proj.scales"],
                sd[p + "post_attention_layernorm.weight"],
                sd[p + "mlp.gate_proj.qweight"], sd[p + "mlp.gate_proj.scales"],
                sd[p + "mlp.up_proj.qweight"], sd[p + "mlp.up_proj.scales"],
                sd[p + "mlp.down_proj.qweight"], sd[p + "mlp.down_proj.scales"]]
        if (p + "self_attn.qkv_proj.bias") in sd:
            caps.append(sd[p + "self_attn.qkv_proj.bias"])
        layers.append(caps)
    return RustQwenDecoder(sd["embed_tokens.weight"], layers, sd["norm.weight"],
                           sd["lm_head.qweight"], sd["lm_head.scales"], cfg["num_hidden_layers"],
                           cfg["hidden_size"], cfg["intermediate_size"],
                           cfg["num_attention_heads"], cfg["num_key_value_heads"],
                           cfg["head_dim"], group_size, cfg["rms_norm_eps"], max_seq_len,
                           cfg["rope_theta"])


def create_decoder_from_checkpoint(model_dir: str, quant: str = "int4", max_seq_len: int = 4096,
                                   device: Optional[torch.device] = None):
    """Local checkpoint -> quantized (or cached) tensors on the device -> decoder."""
    sd, cfg, _ = load_quantized(model_dir, quant, device)
    dec = decoder_from_state_dict(sd, cfg, max_seq_len)
    del sd
    return dec

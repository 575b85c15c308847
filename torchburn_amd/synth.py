"""Seeded synthetic inputs for the benchmark configurations.

Shared by bench.py and the tests so the GPU path and the CPU oracle see the
same bytes.  Distributions follow the benchmark configurations: activations
N(0, 1); INT4 weights uniform in [-8, 7] (so every packed byte is uniform in
[0, 255]); group scales |N(0, 0.02)| + 1e-3; INT8 weights uniform in
[-127, 127] with per-row scales |N(0, 0.02)| / 16 + 1e-4.
"""
from __future__ import annotations

import numpy as np


def rng(seed: int, *stream: int) -> np.random.Generator:
    return np.random.default_rng([seed, *stream])


def activations(g: np.random.Generator, *shape: int) -> np.ndarray:
    return g.standard_normal(shape, dtype=np.float32)


def int4_weight(g: np.random.Generator, n: int, k: int, group_size: int = 32):
    """(packed u8 [n, k/2], scales f32 [n, k/group_size]) in the reference layout."""
    packed = g.integers(0, 256, size=(n, (k + 1) // 2), dtype=np.uint8)
    scales = (np.abs(g.normal(0.0, 0.02, size=(n, k // group_size))) + 1e-3).astype(np.float32)
    return packed, scales


def int8_weight(g: np.random.Generator, n: int, k: int):
    """(i8 [n, k] uniform in [-127, 127], per-row f32 scales [n])."""
    q = g.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = (np.abs(g.normal(0.0, 0.02, size=n)) / 16 + 1e-4).astype(np.float32)
    return q, s


# Model shapes of the benchmark configurations.
QWEN_0_5B = dict(num_layers=24, hidden=896, intermediate=4864, num_heads=14, num_kv_heads=2,
                 head_dim=64, vocab=151936, eps=1e-6, rope_theta=1e6, qkv_bias=True)
LLAMA3_8B = dict(num_layers=32, hidden=4096, intermediate=14336, num_heads=32, num_kv_heads=8,
                 head_dim=128, vocab=128256, eps=1e-5, rope_theta=5e5, qkv_bias=False)


def decoder_weights(cfg: dict, seed: int, wkind: int = 4, lmkind: int = 4,
                    group_size: int = 32) -> dict:
    """Random-init weights of the decoder architecture ``cfg``.

    Layer tensors follow the reference decoder's capsule order
    (src/llm/decoder.rs:260-308): in_norm, qkv_w, qkv_s, o_w, o_s, post_norm,
    gate_w, gate_s, up_w, up_s, down_w, down_s, (qkv_b).  RMSNorm weights are
    1.0, embeddings and an fp32 lm_head N(0, 0.02), qkv bias N(0, 0.02).
    """
    H, I = cfg["hidden"], cfg["intermediate"]
    hq, hkv, hd = cfg["num_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    V = cfg["vocab"]
    tq = (hq + 2 * hkv) * hd

    def proj(g, n, k):
        if wkind == 4:
            return int4_weight(g, n, k, group_size)
        return int8_weight(g, n, k)

    layers = []
    for li in range(cfg["num_layers"]):
        g = rng(seed, 1, li)
        qkv_w, qkv_s = proj(g, tq, H)
        o_w, o_s = proj(g, H, hq * hd)
        gate_w, gate_s = proj(g, I, H)
        up_w, up_s = proj(g, I, H)
        down_w, down_s = proj(g, H, I)
        lw = dict(in_norm=np.ones(H, np.float32), post_norm=np.ones(H, np.float32),
                  qkv_w=qkv_w, qkv_s=qkv_s, o_w=o_w, o_s=o_s, gate_w=gate_w, gate_s=gate_s,
                  up_w=up_w, up_s=up_s, down_w=down_w, down_s=down_s)
        if cfg.get("qkv_bias"):
            lw["qkv_b"] = g.normal(0.0, 0.02, size=tq).astype(np.float32)
        layers.append(lw)
    g = rng(seed, 2)
    embed = g.normal(0.0, 0.02, size=(V, H)).astype(np.float32)
    if lmkind == 4:
        lm_w, lm_s = int4_weight(g, V, H, group_size)
    elif lmkind == 8:
        lm_w, lm_s = int8_weight(g, V, H)
    else:
        lm_w, lm_s = g.normal(0.0, 0.02, size=(V, H)).astype(np.float32), None
    return dict(embed=embed, final_norm=np.ones(H, np.float32), lm_head_w=lm_w, lm_head_s=lm_s,
                layers=layers)


def kv_prefill(cfg: dict, seed: int, seq_len: int, max_seq: int):
    """Per-layer (k, v) f32 [hkv, max_seq, hd] with positions < seq_len ~ N(0, 1)."""
    hkv, hd = cfg["num_kv_heads"], cfg["head_dim"]
    out = []
    for li in range(cfg["num_layers"]):
        g = rng(seed, 3, li)
        k = np.zeros((hkv, max_seq, hd), np.float32)
        v = np.zeros((hkv, max_seq, hd), np.float32)
        k[:, :seq_len] = g.standard_normal((hkv, seq_len, hd), dtype=np.float32)
        v[:, :seq_len] = g.standard_normal((hkv, seq_len, hd), dtype=np.float32)
        out.append((k, v))
    return out


def decoder_weights_torch(cfg: dict, seed: int, wkind: int = 4, lmkind: int = 4,
                          group_size: int = 32, device: str = "cuda") -> dict:
    """decoder_weights() generated directly on a torch device (same layout and
    distributions, torch's generator) -- for multi-GB benchmark models."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    H, I = cfg["hidden"], cfg["intermediate"]
    hq, hkv, hd = cfg["num_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    V = cfg["vocab"]
    tq = (hq + 2 * hkv) * hd

    def normal(shape, std):
        return torch.randn(shape, device=device, generator=g).mul_(std)

    def proj(n, k, bits):
        if bits == 4:
            w = torch.randint(0, 256, (n, (k + 1) // 2), dtype=torch.uint8, device=device,
                              generator=g)
            return w, normal((n, k // group_size), 0.02).abs_().add_(1e-3)
        if bits == 8:
            w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=device, generator=g)
            return w, normal((n,), 0.02).abs_().div_(16).add_(1e-4)
        return normal((n, k), 0.02), None

    layers = []
    for _ in range(cfg["num_layers"]):
        qkv_w, qkv_s = proj(tq, H, wkind)
        o_w, o_s = proj(H, hq * hd, wkind)
        gate_w, gate_s = proj(I, H, wkind)
        up_w, up_s = proj(I, H, wkind)
        down_w, down_s = proj(H, I, wkind)
        lw = dict(in_norm=torch.ones(H, device=device), post_norm=torch.ones(H, device=device),
                  qkv_w=qkv_w, qkv_s=qkv_s, o_w=o_w, o_s=o_s, gate_w=gate_w, gate_s=gate_s,
                  up_w=up_w, up_s=up_s, down_w=down_w, down_s=down_s)
        if cfg.get("qkv_bias"):
            lw["qkv_b"] = normal((tq,), 0.02)
        layers.append(lw)
    lm_w, lm_s = proj(V, H, lmkind)
    return dict(embed=normal((V, H), 0.02), final_norm=torch.ones(H, device=device),
                lm_head_w=lm_w, lm_head_s=lm_s, layers=layers)


def prefill_flops(cfg: dict, n: int, start: int = 0) -> int:
    """Algorithmic FLOPs of prefilling n prompt tokens after `start` cached ones:
    2 per multiply-add of the four projections for every token, QK^T and PV over
    positions 0..p for the token at p, and the lm_head for the last token only."""
    H, I = cfg["hidden"], cfg["intermediate"]
    hq, hkv, hd = cfg["num_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    tq = (hq + 2 * hkv) * hd
    lin = 2 * (tq * H + H * hq * hd + 3 * I * H)
    keys = sum(start + i + 1 for i in range(n))
    attn = 2 * 2 * hq * hd * keys
    return cfg["num_layers"] * (lin * n + attn) + 2 * cfg["vocab"] * H


def decode_bytes_per_token(cfg: dict, pos: int, wkind: int, lmkind: int,
                           group_size: int = 32, v2: bool = False) -> int:
    """Algorithmic HBM bytes of one decoder step at position `pos`: every weight
    byte once (projections, norms, lm_head, one embedding row) plus the KV rows
    0..pos read and the new K/V row written.  v2: QKV, O, down and an INT4
    lm_head are 34-byte blocks per 64 weights (group 64)."""
    H, I = cfg["hidden"], cfg["intermediate"]
    hq, hkv, hd = cfg["num_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    tq = (hq + 2 * hkv) * hd

    def proj(n, k, bits, blocks=False):
        if bits == 4 and blocks:
            return n * (k // 64) * 34
        if bits == 4:
            return n * ((k + 1) // 2) + 4 * n * (k // group_size)
        if bits == 8:
            return n * k + 4 * n
        return 4 * n * k

    layer = (proj(tq, H, wkind, v2) + proj(H, hq * hd, wkind, v2) + 2 * proj(I, H, wkind) +
             proj(H, I, wkind, v2) + 2 * 4 * H + (4 * tq if cfg.get("qkv_bias") else 0))
    kv = 2 * hkv * (pos + 1) * hd * 4 + 2 * hkv * hd * 4
    return (cfg["num_layers"] * (layer + kv) + proj(cfg["vocab"], H, lmkind, v2) + 4 * H + 4 * H)

"""Parity of the gfx950 INT8 per-channel GEMV / SwiGLU MLP with the CPU oracle
(gemv_w8a32, src/quantization/gemv.rs:733-1061; fused_swiglu_mlp_w8a32,
src/quantization/fused_ops.rs:8-133).  Metric max|d| / max|ref| < 1e-4."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from torchburn_amd import synth
import torchburn_amd as tb

pytestmark = pytest.mark.gpu


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (1, 128256, 4096), (2, 1000, 896),
                                   (3, 77, 64), (1, 4096, 14336),
                                   # K slices that end inside a wave's pieces: 152 chunks on
                                   # 3 waves of 51 lanes, 65 chunks on 2 waves of 33
                                   (1, 300, 4864), (2, 77, 2080), (1, 50, 96)])
def test_w8_linear_matches_oracle(cuda, m, n, k):
    print(f"case w8a32_linear m={m} n={n} k={k}", flush=True)
    g = synth.rng(21, m, n, k)
    x = synth.activations(g, m, k)
    w, s = synth.int8_weight(g, n, k)
    b = g.normal(0, 0.1, n).astype(np.float32)
    ref = O.gemv_w8(x, w, s, b)
    T = lambda a: torch.from_numpy(a).to(cuda)
    y = tb.w8a32_linear(T(x), T(w), T(s), T(b)).cpu().numpy()
    assert rel(y, ref) < 1e-4


def test_w8_per_tensor_scale(cuda):
    g = synth.rng(22)
    x = synth.activations(g, 1, 512)
    w, _ = synth.int8_weight(g, 64, 512)
    s = np.array([0.03], np.float32)
    T = lambda a: torch.from_numpy(a).to(cuda)
    y = tb.w8a32_linear(T(x), T(w), T(s)).cpu().numpy()
    assert rel(y, O.gemv_w8(x, w, s)) < 1e-4


@pytest.mark.parametrize("m,k,inter,bias,scalar", [
    (1, 1024, 2048, False, ""),          # per-row scales, no biases
    (1, 1024, 2048, True, ""),           # biases on gate, up and down
    (1, 1024, 2048, True, "gud"),        # one per-tensor scale on every projection
    (3, 512, 1536, True, "g"),           # mixed: scalar gate scale, per-row up / down
    (2, 4096, 14336, False, "d"),        # Llama-3-8B MLP shape, scalar down scale
])
def test_w8_swiglu_mlp_matches_oracle(cuda, m, k, inter, bias, scalar):
    """fused_swiglu_mlp_w8a32 (fused_ops.rs:8-133) with the reference's optional
    biases and its per-tensor scale branch (gs_len == 1, fused_ops.rs:80-97)."""
    print(f"case w8 swiglu mlp m={m} k={k} inter={inter} bias={bias} scalar={scalar}", flush=True)
    g = synth.rng(23, m, k, inter)
    x = synth.activations(g, m, k)
    gw, gsc = synth.int8_weight(g, inter, k)
    uw, usc = synth.int8_weight(g, inter, k)
    dw, dsc = synth.int8_weight(g, k, inter)
    one = lambda s: s[:1].copy()
    gsc = one(gsc) if "g" in scalar else gsc
    usc = one(usc) if "u" in scalar else usc
    dsc = one(dsc) if "d" in scalar else dsc
    nb = lambda n: g.normal(0, 0.1, n).astype(np.float32) if bias else None
    gb, ub, db = nb(inter), nb(inter), nb(k)
    ref = O.swiglu_mlp_w8(x, gw, gsc, uw, usc, dw, dsc, gb=gb, ub=ub, db=db)
    T = lambda a: None if a is None else torch.from_numpy(a).to(cuda)
    out = tb.fused_swiglu_mlp_w8a32(T(x), T(gw), T(gsc), T(gb), T(uw), T(usc), T(ub), T(dw),
                                    T(dsc), T(db)).cpu().numpy()
    assert rel(out, ref) < 1e-4


def test_w8_swiglu_mlp_rejects_bad_scales(cuda):
    """A scale vector that is neither per-tensor nor per-row is refused before
    any device read (the kernel would otherwise read past it)."""
    g = synth.rng(24)
    x = synth.activations(g, 1, 256)
    gw, gsc = synth.int8_weight(g, 512, 256)
    uw, usc = synth.int8_weight(g, 512, 256)
    dw, dsc = synth.int8_weight(g, 256, 512)
    T = lambda a: torch.from_numpy(a).to(cuda)
    with pytest.raises(tb.UnsupportedOpError):
        tb.fused_swiglu_mlp_w8a32(T(x), T(gw), T(gsc[:7]), None, T(uw), T(usc), None, T(dw),
                                  T(dsc), None)
    with pytest.raises(tb.UnsupportedOpError):
        tb.fused_swiglu_mlp_w8a32(T(x), T(gw[:, :128]), T(gsc), None, T(uw), T(usc), None,
                                  T(dw), T(dsc), None)

"""Shapes beyond the streaming kernels, and the per-channel INT4 entry points.

* per-channel w4a32_linear (reference gemv.rs:1066-1182, the compile engine's
  d_quant.rs:109-125) and quantize_weight_int4 (fused_ops.rs:592-639) against
  the oracle's restatements (orc_gemv_w4_rows, orc_quantize_int4_rows);
* grouped INT4 / INT8 projections and fused MLPs at K not a multiple of 32,
  group sizes other than 32 / 64, and K past one GEMV pass (the reference takes
  all of them, gemv.rs:1650-1660), through the any-shape GEMV or the streaming
  kernels, against the oracle (orc_gemm_w4, orc_gemv_w8, the MLP restatements);
* fused_swiglu_mlp_batched over QuantizedLinear modules (quantization.py:358-405).
Metric max|d| / max|ref| < 1e-4; quantizers bit-exact.
"""
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


def T(a, dev):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("m,n,k,scalar", [
    (1, 4096, 4096, False),     # streaming GEMV, one scale per row
    (3, 300, 896, False),       # GEMV pass of 3 rows
    (7, 512, 4096, True),       # FP32-MFMA projection, one per-tensor scale
    (1, 77, 1001, False),       # odd K: any-shape GEMV
    (2, 50, 31, True),          # K below one chunk
    (1, 256, 20480, False),     # K past one GEMV pass
    (24, 512, 4096, False),     # limb GEMM (M >= 17), one scale per row
    (40, 300, 1024, True),      # limb GEMM, one per-tensor scale, ragged N
    (16, 1000, 4064, False),    # FP32-MFMA projection (K % 128 != 0), one scale per row
    (9, 300, 2080, True),       # FP32-MFMA projection (K % 128 != 0), one per-tensor scale
])
def test_w4a32_linear_per_channel(cuda, m, n, k, scalar):
    print(f"case w4a32_linear m={m} n={n} k={k} scalar={scalar}", flush=True)
    g = synth.rng(41, m, n, k)
    x = synth.activations(g, m, k)
    q = g.integers(-8, 8, (n, k)).astype(np.int8)
    w = O.pack_int4(q)
    s = (np.abs(g.normal(0, 0.02, 1 if scalar else n)) + 1e-3).astype(np.float32)
    b = g.normal(0, 0.1, n).astype(np.float32)
    ref = O.gemv_w4_rows(x, w, s, b)
    y = tb.w4a32_linear(T(x, cuda), T(w, cuda), T(s, cuda), T(b, cuda)).cpu().numpy()
    assert y.shape == (m, n)
    assert rel(y, ref) < 1e-4


@pytest.mark.parametrize("n,k", [(64, 4096), (33, 1001), (7, 2)])
def test_quantize_weight_int4_bit_exact(cuda, n, k):
    print(f"case quantize_weight_int4 n={n} k={k}", flush=True)
    g = synth.rng(42, n, k)
    w = (g.standard_normal((n, k)) * 0.05).astype(np.float32)
    w[0, : min(k, 3)] = [0.7, 0.35, -0.35][: min(k, 3)]   # ties at scale 0.1
    if n > 3:
        w[3] = 0.0
    qr, sr = O.quantize_int4_rows(w)
    q, s = tb.quantize_weight_int4(T(w, cuda))
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(s.cpu().numpy(), sr)
    with pytest.raises(ValueError):
        tb.quantize_weight_int4(torch.randn(16, device=cuda))


def test_quantize_weight_int4_non_finite(cuda):
    """NaN and infinite weights give the reference's nibbles (NaN -> 8; an
    infinite weight zeroes its row), bit-exact against the oracle."""
    print("case quantize_weight_int4 non-finite", flush=True)
    w = np.float32([[np.nan, 1.0, -7.0, 7.0], [np.inf, 1.0, -2.0, 0.5], [-np.inf, np.nan, 3.0, 0.0]])
    qr, sr = O.quantize_int4_rows(w)
    q, s = tb.quantize_weight_int4(T(w, cuda))
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(s.cpu().numpy(), sr)


@pytest.mark.parametrize("m,n,k,gs", [
    (1, 300, 1000, 40),     # group 40, K % 32 != 0
    (2, 256, 4096, 128),    # power-of-two group 128 on the streaming GEMV
    (6, 256, 4096, 128),    # ... and on the MFMA projection
    (1, 128, 28672, 32),    # K past one GEMV pass (Llama-70B intermediate)
    (1, 64, 1001, 32),      # odd K, short last group
    (5, 96, 100, 20),       # 5 rows, odd shape: any-shape GEMV
    (40, 256, 4096, 128),   # group 128 on the limb GEMM (M >= 17)
    (18, 130, 384, 64),     # group 64, two slabs (one of 2 rows), ragged N
])
def test_w4_grouped_general_shapes(cuda, m, n, k, gs):
    print(f"case w4a32_grouped_linear m={m} n={n} k={k} gs={gs}", flush=True)
    g = synth.rng(43, m, n, k, gs)
    x = synth.activations(g, m, k)
    q = g.integers(-8, 8, (n, k)).astype(np.int8)
    w = O.pack_int4(q)
    ng = (k + gs - 1) // gs
    s = (np.abs(g.normal(0, 0.02, (n, ng))) + 1e-3).astype(np.float32)
    b = g.normal(0, 0.1, n).astype(np.float32)
    ref = O.gemm_w4(x, w, s, b, group_size=gs)
    y = tb.w4a32_grouped_linear(T(x, cuda), T(w, cuda), T(s, cuda), T(b, cuda),
                                group_size=gs).cpu().numpy()
    assert rel(y, ref) < 1e-4


def test_w4_odd_group_refused(cuda):
    x = torch.randn(1, 90, device=cuda)
    w = torch.zeros(4, 45, dtype=torch.uint8, device=cuda)
    s = torch.ones(4, 10, device=cuda)
    with pytest.raises(tb.UnsupportedOpError, match="even"):
        tb.w4a32_grouped_linear(x, w, s, None, group_size=9)


@pytest.mark.parametrize("m,n,k", [(1, 100, 1000), (3, 50, 17), (1, 64, 20000)])
def test_w8_general_shapes(cuda, m, n, k):
    print(f"case w8a32_linear m={m} n={n} k={k}", flush=True)
    g = synth.rng(44, m, n, k)
    x = synth.activations(g, m, k)
    w, s = synth.int8_weight(g, n, k)
    b = g.normal(0, 0.1, n).astype(np.float32)
    ref = O.gemv_w8(x, w, s, b)
    y = tb.w8a32_linear(T(x, cuda), T(w, cuda), T(s, cuda), T(b, cuda)).cpu().numpy()
    assert rel(y, ref) < 1e-4


@pytest.mark.parametrize("m,k,inter,gs", [
    (1, 4096, 28672, 32),   # down K = 28672: past one GEMV pass
    (2, 1000, 520, 40),     # odd shapes throughout
])
def test_w4_mlp_general_shapes(cuda, m, k, inter, gs):
    print(f"case fused_swiglu_mlp_w4a32 m={m} k={k} inter={inter} gs={gs}", flush=True)
    g = synth.rng(45, m, k, inter)
    x = synth.activations(g, m, k)

    def wq(n, kk):
        q = g.integers(-8, 8, (n, kk)).astype(np.int8)
        ng = (kk + gs - 1) // gs
        return O.pack_int4(q), (np.abs(g.normal(0, 0.02, (n, ng))) + 1e-3).astype(np.float32)

    gw, gsc = wq(inter, k)
    uw, usc = wq(inter, k)
    dw, dsc = wq(k, inter)
    gb = g.normal(0, 0.1, inter).astype(np.float32)
    ref = O.swiglu_mlp_w4(x, gw, gsc, uw, usc, dw, dsc, gb=gb, group_size=gs)
    out = tb.fused_swiglu_mlp_w4a32(T(x, cuda), T(gw, cuda), T(gsc, cuda), T(gb, cuda),
                                    T(uw, cuda), T(usc, cuda), None, T(dw, cuda), T(dsc, cuda),
                                    None, gs).cpu().numpy()
    assert rel(out, ref) < 1e-4


def test_w8_mlp_odd_k(cuda):
    print("case fused_swiglu_mlp_w8a32 m=2 k=1000 inter=2000", flush=True)
    g = synth.rng(46)
    m, k, inter = 2, 1000, 2000
    x = synth.activations(g, m, k)
    gw, gsc = synth.int8_weight(g, inter, k)
    uw, usc = synth.int8_weight(g, inter, k)
    dw, dsc = synth.int8_weight(g, k, inter)
    ub = g.normal(0, 0.1, inter).astype(np.float32)
    ref = O.swiglu_mlp_w8(x, gw, gsc, uw, usc, dw, dsc[:1].copy(), ub=ub)
    out = tb.fused_swiglu_mlp_w8a32(T(x, cuda), T(gw, cuda), T(gsc, cuda), None, T(uw, cuda),
                                    T(usc, cuda), T(ub, cuda), T(dw, cuda),
                                    T(dsc[:1].copy(), cuda), None).cpu().numpy()
    assert rel(out, ref) < 1e-4


@pytest.mark.parametrize("tokens", [1, 6, 20])
def test_fused_swiglu_mlp_batched_modules(cuda, tokens):
    """fused_swiglu_mlp_batched(x, gate, up, down) over QuantizedLinear modules, as
    the reference's model.py:359 calls it during prefill."""
    print(f"case fused_swiglu_mlp_batched tokens={tokens}", flush=True)
    torch.manual_seed(tokens)
    k, inter = 512, 1024
    lin = [torch.nn.Linear(k, inter, bias=False), torch.nn.Linear(k, inter, bias=False),
           torch.nn.Linear(inter, k, bias=False)]
    gate, up, down = (tb.QuantizedLinear.from_float(l, bits=4, group_size=64) for l in lin)
    x = torch.randn(1, tokens, k)
    out = tb.fused_swiglu_mlp_batched(x, gate, up, down)
    assert out.shape == (1, tokens, k)
    n = lambda t: t.detach().cpu().numpy()
    ref = O.swiglu_mlp_w4(n(x).reshape(tokens, k), n(gate.qweight), n(gate.scales),
                          n(up.qweight), n(up.scales), n(down.qweight), n(down.scales),
                          group_size=64)
    assert rel(n(out).reshape(tokens, k), ref) < 1e-4
    q8 = [tb.QuantizedLinear.from_float(l, bits=8) for l in lin]
    out8 = tb.fused_swiglu_mlp_batched(x, *q8)
    ref8 = O.swiglu_mlp_w8(n(x).reshape(tokens, k), n(q8[0].qweight), n(q8[0].scales),
                           n(q8[1].qweight), n(q8[1].scales), n(q8[2].qweight), n(q8[2].scales))
    assert rel(n(out8).reshape(tokens, k), ref8) < 1e-4

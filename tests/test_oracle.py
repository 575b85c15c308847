"""Pins the CPU oracle (oracle/tb_oracle.c) before it is trusted as the checker.

What pins each oracle function (no golden-vector files exist in the reference;
its own tests recompute expectations in-test, so their deterministic inputs and
budgets are reproduced here):

  pack / unpack      all 256 byte values; random round trips; the reference's
                     quantize_grouped KAT (tests/parity/int4.rs:12-38)
  quantizer          numpy closed form with half-to-even rounding
                     (python/torchburn/quantization.py:53-118)
  gemv_w4 / gemm_w4  float64 brute force (tests/parity/int4.rs:109-126), the
                     reference's KAT inputs and budgets (int4.rs:172-255, 303-329),
                     special cases (x = 0, constant q, one-hot x)
  swiglu             float64 closed form via torch.nn.functional.silu
  gemv_w8            the dot_f32_i8 KAT (tests/parity/int8.rs:24-37), float64,
                     quality budget (int8.rs:41-67)
  swiglu_w8          float64 closed form with biases, per-row and per-tensor
                     scales (fused_ops.rs:8-133); a dropped bias or a per-row
                     read of a scalar scale fails it
  gemv_w4_rows       per-channel w4a32_linear (gemv.rs:1066-1182): float64 with
                     odd K and short K, per-row and scalar scales, bias;
                     one-hot x returns (q - 8) * s exactly
  quantize_int4_rows numpy closed form, ties away from zero, odd-K padding
                     nibble 8, zero rows -> scale 1 (fused_ops.rs:592-639)
  gemv_f32           float64; one-hot x returns a column exactly; integer
                     weights and x = 1 give exact row sums
  quantize_int8      numpy closed form with ties away from zero and the 1e-8
                     zero-row threshold (fused_ops.rs:554-589)
  rms_norm           the reference's KAT (tests/parity/decoder.rs:14-29) and
                     torch.nn.functional.rms_norm in float64
  rms_norm_torch     torch.nn.functional.rms_norm in float32 on the CPU (the
                     per-layer path's own op) within 2 ulp, and float64
  rope               RoPE as a complex rotation in float64 (a different formula),
                     pos 0 is the identity, pair norms preserved
  attention          torch scaled_dot_product_attention(enable_gqa) in float64;
                     seq_len 1 returns v; identical keys give mean(V); the same
                     for the per-layer steps' variant (attention_layer)
  argmax             decoder.rs:32-40 KAT, ties -> lowest index
  f32 RoPE tables    (torchburn_amd.decoder.rotary_tables_f32, the per-layer
                     path's tables) cos / sin of the float32 angle within 1 ulp,
                     the angle within f32 rounding of pos * theta^(-2i/d)
  decoder step       an independent float64 torch model built from library ops
                     (rms_norm, complex RoPE, SDPA, silu) on a small config, for
                     INT4 and INT8 projections and INT4 / INT8 / fp32 lm_heads,
                     and with caller tables + the per-layer numerics; at
                     group 64 with every dimension a multiple of 64 the model uses
                     binary16-rounded QKV / O / down / lm_head scales (the
                     reference's v2 repack) and the f32-scale model is shown to differ
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O
from torchburn_amd import synth


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-6))


def dequant(w, s, k, gs):
    q = O.unpack_int4(w, k).astype(np.float64)
    return q * np.repeat(s.astype(np.float64), gs, axis=1)[:, :k]


# ---------------------------------------------------------------- packing ---

def test_unpack_all_bytes():
    w = np.arange(256, dtype=np.uint8).reshape(1, 256)
    q = O.unpack_int4(w, 512)[0]
    b = np.arange(256)
    assert np.array_equal(q[0::2], (b & 15) - 8)
    assert np.array_equal(q[1::2], (b >> 4) - 8)


@pytest.mark.parametrize("k", [2, 31, 32, 896, 1001])
def test_pack_round_trip(k):
    q = np.random.default_rng(k).integers(-8, 8, size=(7, k), dtype=np.int8)
    w = O.pack_int4(q)
    assert w.shape == (7, (k + 1) // 2)
    assert np.array_equal(O.unpack_int4(w, k), q)
    # byte j = (q[2j] + 8) | (q[2j+1] + 8) << 4
    assert int(w[0, 0]) == (int(q[0, 0]) + 8) | ((int(q[0, 1]) + 8) << 4)


@pytest.mark.parametrize("k,gs", [(128, 32), (384, 128), (96, 3), (200, 100), (10, 1)])
def test_quantizer_matches_closed_form(k, gs):
    g = np.random.default_rng(3)
    w = g.normal(0, 1, (9, k)).astype(np.float32)
    w[0, :gs] = 0.0                      # all-zero group -> scale 1e-8
    w[1, min(5, gs - 1)] = 3.5 * (np.abs(w[1, :gs]).max() / 7.0)   # an exact .5 tie
    packed, scales = O.quantize_int4_grouped(w, gs)
    wg = w.reshape(9, k // gs, gs)
    s = np.maximum(np.abs(wg).max(-1) / np.float32(7.0), np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.round(wg / s[..., None]), -8, 7).astype(np.int8).reshape(9, k)
    assert np.array_equal(scales, s)
    assert np.array_equal(packed, O.pack_int4(q))


def reference_quantize_grouped(w, k, gs):
    """tests/parity/int4.rs:12-38: scale = max_abs/7 (1.0 if <= 1e-8), q = round-half-away."""
    n = w.size // k
    wg = w.reshape(n, k // gs, gs)
    mx = np.abs(wg).max(-1)
    s = np.where(mx > 1e-8, mx / np.float32(7.0), np.float32(1.0)).astype(np.float32)
    v = wg * (np.float32(1.0) / s)[..., None]
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -8, 7).astype(np.int8)
    return O.pack_int4(q.reshape(n, k)), s


# ------------------------------------------------------------------- gemv ---

@pytest.mark.parametrize("n,k,gs", [(64, 896, 32), (64, 896, 64), (33, 4096, 32),
                                    (5, 96, 32), (8, 48, 16), (3, 40, 8)])
def test_gemv_w4_vs_float64(n, k, gs):
    g = np.random.default_rng(n * k + gs)
    x = g.standard_normal((2, k), dtype=np.float32)
    w = g.integers(0, 256, (n, (k + 1) // 2), dtype=np.uint8)
    s = (np.abs(g.normal(0, 0.02, (n, k // gs))) + 1e-3).astype(np.float32)
    b = g.normal(0, 0.1, n).astype(np.float32)
    y = O.gemm_w4(x, w, s, b, group_size=gs)
    ref = x.astype(np.float64) @ dequant(w, s, k, gs).T + b
    assert rel(y, ref) < 1e-6
    assert np.allclose(O.gemv_w4_f64(x[0], w, s, b, gs), ref[0], rtol=1e-12, atol=1e-12)


def test_gemv_w4_reference_kat():
    """tests/parity/int4.rs:172-215 inputs; the oracle is the exact-W4A32 tier."""
    n, k, gs = 64, 896, 64
    x = (np.sin(np.arange(k, dtype=np.float32) * np.float32(0.13)) * 2).astype(np.float32)
    w = (np.cos(np.arange(n * k, dtype=np.float32) * np.float32(0.29)) * 1.5).astype(np.float32)
    packed, scales = reference_quantize_grouped(w, k, gs)
    y = O.gemm_w4(x[None], packed, scales, group_size=gs)[0]
    ref = x.astype(np.float64) @ dequant(packed, scales, k, gs).T
    assert rel(y, ref) < 1e-3          # the reference's budget
    assert rel(y, ref) < 1e-6          # and the oracle's own


def test_gemv_w4_quality_budget():
    """tests/parity/int4.rs:221-255: int4-g64 vs unquantized f32 < 0.2."""
    n, k = 32, 512
    x = (np.cos(np.arange(k, dtype=np.float32) * np.float32(0.07)) * 1.2).astype(np.float32)
    w = (np.sin(np.arange(n * k, dtype=np.float32) * np.float32(0.17)) * 2).astype(np.float32)
    packed, scales = reference_quantize_grouped(w, k, 64)
    y = O.gemm_w4(x[None], packed, scales, group_size=64)[0]
    assert rel(y, w.reshape(n, k).astype(np.float64) @ x) < 0.2


def test_gemv_w4_bias_kat():
    """tests/parity/int4.rs:303-329."""
    n, k = 16, 64
    x = np.full(k, 0.5, np.float32)
    w = (np.sin(np.arange(n * k, dtype=np.float32) * np.float32(0.23)) * 0.5).astype(np.float32)
    packed, scales = reference_quantize_grouped(w, k, 64)
    bias = (np.arange(n) * 0.01 + 0.1).astype(np.float32)
    y = O.gemm_w4(x[None], packed, scales, bias, group_size=64)[0]
    want = x.astype(np.float64) @ dequant(packed, scales, k, 64).T + bias
    assert np.all(np.abs(y - want) / np.maximum(np.abs(want), 1e-4) < 1e-2)


def test_gemv_w4_special_cases():
    n, k = 24, 128
    g = np.random.default_rng(1)
    w = g.integers(0, 256, (n, k // 2), dtype=np.uint8)
    s = g.uniform(0.5, 2, (n, k // 32)).astype(np.float32)
    b = g.normal(0, 1, n).astype(np.float32)
    assert np.array_equal(O.gemm_w4(np.zeros((1, k), np.float32), w, s, b, group_size=32)[0], b)
    x = g.standard_normal((1, k), dtype=np.float32)
    for c in (-8, 0, 7):
        wc = np.full((n, k // 2), (c + 8) | ((c + 8) << 4), np.uint8)
        y = O.gemm_w4(x, wc, np.ones((n, k // 32), np.float32), group_size=32)[0]
        assert np.allclose(y, c * x.astype(np.float64).sum(), rtol=1e-5, atol=1e-5)
    q = O.unpack_int4(w, k)
    for col in (0, 1, 63, 127):
        e = np.zeros((1, k), np.float32)
        e[0, col] = 1
        y = O.gemm_w4(e, w, s, group_size=32)[0]
        assert np.array_equal(y, q[:, col].astype(np.float32) * s[:, col // 32])


def test_swiglu_mlp_vs_float64():
    g = np.random.default_rng(4)
    m, k, inter = 2, 128, 96
    x = g.standard_normal((m, k), dtype=np.float32)
    gw, gsc = synth.int4_weight(g, inter, k, 32)
    uw, usc = synth.int4_weight(g, inter, k, 32)
    dw, dsc = synth.int4_weight(g, k, inter, 32)
    gb = g.normal(0, 0.1, inter).astype(np.float32)
    out = O.swiglu_mlp_w4(x, gw, gsc, uw, usc, dw, dsc, gb=gb, group_size=32)
    xd = torch.from_numpy(x.astype(np.float64))
    gg = xd @ torch.from_numpy(dequant(gw, gsc, k, 32)).T + torch.from_numpy(gb.astype(np.float64))
    uu = xd @ torch.from_numpy(dequant(uw, usc, k, 32)).T
    h = F.silu(gg) * uu
    ref = (h @ torch.from_numpy(dequant(dw, dsc, inter, 32)).T).numpy()
    assert rel(out, ref) < 1e-5


@pytest.mark.parametrize("k", [1000, 7, 64])
def test_gemv_f32_vs_float64(k):
    """orc_gemv_f32 (fp32 lm_head, model.py:499-500): float64, exact special cases.
    k = 1000 ends in an 8-element tail, k = 7 takes the scalar branch."""
    g = np.random.default_rng(k)
    n = 37
    x = g.standard_normal(k).astype(np.float32)
    w = g.standard_normal((n, k)).astype(np.float32)
    assert rel(O.gemv_f32(x, w), w.astype(np.float64) @ x.astype(np.float64)) < 1e-6
    for j in (0, k // 2, k - 1):
        e = np.zeros(k, np.float32)
        e[j] = 1.0
        assert np.array_equal(O.gemv_f32(e, w), w[:, j])
    wi = g.integers(-50, 50, (n, k)).astype(np.float32)
    assert np.array_equal(O.gemv_f32(np.ones(k, np.float32), wi), wi.sum(1))


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("scalar", ["", "gud", "u"])
def test_swiglu_w8_vs_float64(bias, scalar):
    """fused_swiglu_mlp_w8a32 (fused_ops.rs:8-133): g = dot * gs + gb,
    u = dot * us + ub (a 1-element scale is one per-tensor scalar,
    fused_ops.rs:80-97), h = silu(g) * u, out = dot(h, down) * ds + db."""
    g = np.random.default_rng(11 + bias + len(scalar))
    m, k, inter = 2, 160, 96
    x = g.standard_normal((m, k)).astype(np.float32)
    gw, gsc = synth.int8_weight(g, inter, k)
    uw, usc = synth.int8_weight(g, inter, k)
    dw, dsc = synth.int8_weight(g, k, inter)
    gsc = gsc[:1].copy() if "g" in scalar else gsc
    usc = usc[:1].copy() if "u" in scalar else usc
    dsc = dsc[:1].copy() if "d" in scalar else dsc
    nb = (lambda n: g.normal(0, 0.5, n).astype(np.float32)) if bias else (lambda n: None)
    gb, ub, db = nb(inter), nb(inter), nb(k)
    D = lambda a: np.asarray(a, np.float64)
    z = lambda b, n: np.zeros(n) if b is None else D(b)
    sc = lambda s, n: np.broadcast_to(D(s), (n,))
    ref = []
    for r in range(m):
        gg = (D(gw) @ D(x[r])) * sc(gsc, inter) + z(gb, inter)
        uu = (D(uw) @ D(x[r])) * sc(usc, inter) + z(ub, inter)
        h = F.silu(torch.from_numpy(gg)).numpy() * uu
        assert rel(O.swiglu_h_w8(x[r], gw, gsc, uw, usc, gb, ub), h) < 1e-5
        ref.append((D(dw) @ h) * sc(dsc, k) + z(db, k))
    out = O.swiglu_mlp_w8(x, gw, gsc, uw, usc, dw, dsc, gb=gb, ub=ub, db=db)
    assert rel(out, np.stack(ref)) < 1e-5


@pytest.mark.parametrize("k,scalar", [(896, False), (1001, False), (31, True), (4096, True)])
def test_gemv_w4_rows_vs_float64(k, scalar):
    """Per-channel w4a32_linear: y = dot_f32_u4(x, row) * s + b."""
    g = np.random.default_rng(k)
    n = 45
    q = g.integers(-8, 8, (n, k)).astype(np.int8)
    w = O.pack_int4(q)
    s = (np.abs(g.normal(0, 0.02, 1 if scalar else n)) + 1e-3).astype(np.float32)
    b = g.normal(0, 0.1, n).astype(np.float32)
    x = g.standard_normal((2, k)).astype(np.float32)
    y = O.gemv_w4_rows(x, w, s, b)
    ref = (x.astype(np.float64) @ q.astype(np.float64).T) * np.broadcast_to(s, (n,)) + b
    assert rel(y, ref) < 1e-6
    for j in (0, k - 1):
        e = np.zeros((1, k), np.float32)
        e[0, j] = 1.0
        assert np.array_equal(O.gemv_w4_rows(e, w, s)[0],
                              (q[:, j].astype(np.float32) * np.broadcast_to(s, (n,))))


def test_quantize_int4_rows_closed_form():
    """quantize_linear_weights_int4 (fused_ops.rs:592-639)."""
    g = np.random.default_rng(9)
    n, k = 5, 37                                   # odd K: last byte padded with 8
    w = g.standard_normal((n, k)).astype(np.float32)
    w[1] = 0.0                                     # amax 0 -> scale 1, q 0
    w[2, :3] = [7.0, 3.5, -3.5]                    # scale 1: ties away from zero
    w[2, 3:] = 0.0
    q, s = O.quantize_int4_rows(w)
    amax = np.abs(w).max(1)
    s_want = np.where(amax > np.float32(1e-8), amax / np.float32(7.0), np.float32(1.0))
    assert np.array_equal(s, s_want.astype(np.float32))
    t = (w * (np.float32(1.0) / s_want.astype(np.float32))[:, None]).astype(np.float32)
    t = t.astype(np.float64)
    r = np.clip(np.where(t >= 0, np.floor(t + 0.5), np.ceil(t - 0.5)), -8, 7).astype(np.int8)
    assert np.array_equal(O.unpack_int4(q, k), r)
    assert np.all((q[:, -1] >> 4) == 8)
    assert list(O.unpack_int4(q, k)[2, :3]) == [7, 4, -4] and not O.unpack_int4(q, k)[1].any()


def test_quantize_int4_rows_non_finite():
    """A NaN skips the row maximum (`a > max_abs` is false), survives round and
    clamp, and `as i8` makes it 0: nibble 8.  An infinite weight makes the scale
    infinite and inv 0, so every element of its row becomes 0 * w: NaN for the
    infinite one (nibble 8), 0 for the rest (fused_ops.rs:607-629)."""
    w = np.float32([[np.nan, 1.0, -7.0, 7.0], [np.inf, 1.0, -2.0, 0.5], [-np.inf, np.nan, 3.0, 0.0]])
    q, s = O.quantize_int4_rows(w)
    assert s[0] == 1.0 and np.isinf(s[1]) and np.isinf(s[2])
    assert O.unpack_int4(q, 4).tolist() == [[0, 1, -7, 7], [0, 0, 0, 0], [0, 0, 0, 0]]
    assert q[0, 0] & 15 == 8


# ------------------------------------------------------------------- int8 ---

def test_dot_i8_reference_kat():
    """tests/parity/int8.rs:24-37 (row dot with unit scale)."""
    i = np.arange(2048)
    x = (np.cos(i.astype(np.float32) * np.float32(0.041)) * 2).astype(np.float32)
    w = (((i * 31) % 251) - 125).astype(np.int8)[None]
    got = O.gemv_w8(x[None], w, np.ones(1, np.float32))[0, 0]
    want = float(np.dot(x.astype(np.float64), w[0].astype(np.float64)))
    assert abs(got - want) / max(abs(want), 1e-6) < 1e-3
    assert abs(got - want) / max(abs(want), 1e-6) < 1e-5


def test_gemv_w8_vs_float64_and_quality():
    g = np.random.default_rng(5)
    n, k = 40, 1000       # k % 32 != 0 exercises the 16-wide and scalar tails
    x = g.standard_normal((1, k), dtype=np.float32)
    q, s = synth.int8_weight(g, n, k)
    b = g.normal(0, 0.1, n).astype(np.float32)
    y = O.gemv_w8(x, q, s, b)[0]
    ref = (q.astype(np.float64) @ x[0].astype(np.float64)) * s + b
    assert rel(y, ref) < 1e-6
    # int8.rs:41-67 quality budget, with the oracle's quantizer
    n, k = 32, 512
    xx = (np.cos(np.arange(k, dtype=np.float32) * np.float32(0.051)) * 1.1).astype(np.float32)
    ww = (np.sin(np.arange(n * k, dtype=np.float32) * np.float32(0.19)) * 1.8).astype(np.float32)
    qq, ss = O.quantize_int8(ww.reshape(n, k))
    y = O.gemv_w8(xx[None], qq, ss)[0]
    assert rel(y, ww.reshape(n, k).astype(np.float64) @ xx) < 0.05


def test_quantize_int8_closed_form():
    """fused_ops.rs:554-589: s = amax / 127 (1 when amax <= 1e-8); q = round half
    away from zero of w * (1 / s), clamped to +-127."""
    g = np.random.default_rng(8)
    w = g.standard_normal((6, 96)).astype(np.float32)
    w[1] = 0.0                                  # amax 0 -> scale 1
    w[2] = np.float32(5e-9) * np.sign(w[2])     # amax <= 1e-8 -> scale 1, q 0
    w[3, :4] = [127.0, 2.5, -2.5, 0.5]          # scale 1: ties away from zero
    w[3, 4:] = 0.0
    q, s = O.quantize_int8(w)
    amax = np.abs(w).max(1)
    s_want = np.where(amax > np.float32(1e-8), amax / np.float32(127.0), np.float32(1.0))
    assert np.array_equal(s, s_want.astype(np.float32))
    t = (w * (np.float32(1.0) / s_want.astype(np.float32))[:, None]).astype(np.float32)
    t = t.astype(np.float64)
    r = np.where(t >= 0, np.floor(t + 0.5), np.ceil(t - 0.5))
    assert np.array_equal(q, np.clip(r, -127, 127).astype(np.int8))
    assert list(q[3, :4]) == [127, 3, -3, 1] and not q[2].any()


# -------------------------------------------------------- norm, rope, attn ---

def test_rms_norm_reference_kat():
    """tests/parity/decoder.rs:14-29 inputs and budget."""
    n = 896
    x = (np.sin(np.arange(n, dtype=np.float32) * np.float32(0.31)) * 3).astype(np.float32)
    w = (1 + np.arange(n, dtype=np.float32) * np.float32(0.001)).astype(np.float32)
    out = O.rms_norm(x, w, 1e-6)
    want = F.rms_norm(torch.from_numpy(x.astype(np.float64)), (n,),
                      torch.from_numpy(w.astype(np.float64)), eps=1e-6).numpy()
    assert np.max(np.abs(out - want) / np.maximum(np.abs(want), 1e-6)) < 1e-4
    assert rel(out, want) < 1e-6


@pytest.mark.parametrize("n", [896, 4096, 100])
def test_rms_norm_torch_vs_f_rms_norm(n):
    """orc_rms_norm_torch is the per-layer path's F.rms_norm (model.py:91-98):
    within 2 ulp of torch's own float32 result, and of float64."""
    g = np.random.default_rng(n)
    x = (g.standard_normal(n) * 2).astype(np.float32)
    w = (1 + g.standard_normal(n) * 0.1).astype(np.float32)
    out = O.rms_norm_torch(x, w, 1e-5)
    t32 = F.rms_norm(torch.from_numpy(x), (n,), torch.from_numpy(w), eps=1e-5).numpy()
    ulp = np.spacing(np.abs(t32).astype(np.float32))
    assert np.all(np.abs(out - t32) <= 2 * ulp)
    t64 = F.rms_norm(torch.from_numpy(x.astype(np.float64)), (n,),
                     torch.from_numpy(w.astype(np.float64)), eps=1e-5).numpy()
    assert rel(out, t64) < 1e-6


def test_rotary_tables_f32():
    """The per-layer path's tables: cos / sin of the float32 angle pos * inv_freq
    (model.py:108-122), against float64 mathematics -- and visibly not the
    native decoder's f64 tables at thousands of positions."""
    from torchburn_amd.decoder import rotary_tables_f32
    hd, theta, max_seq = 128, 5e5, 4200
    c, s = rotary_tables_f32(max_seq, hd, theta)
    assert c.dtype == np.float32 and c.shape == (max_seq, hd)
    half = hd // 2
    assert np.array_equal(c[:, :half], c[:, half:]) and np.array_equal(s[:, :half], s[:, half:])
    freq64 = theta ** (-(2.0 * np.arange(half)) / hd)
    pos32 = np.arange(max_seq, dtype=np.float32)
    one = np.spacing(np.float32(1)) * 1.01
    for i in range(half):
        # some float32 inv_freq within 3 ulp of theta^(-2i/d) reproduces the whole
        # column as cos / sin (within 1 ulp) of the float32 product pos * inv_freq
        up, dn = [np.float32(freq64[i])], [np.float32(freq64[i])]
        for _ in range(3):
            up.append(np.nextafter(up[-1], np.float32(np.inf)))
            dn.append(np.nextafter(dn[-1], np.float32(-np.inf)))
        cands = up + dn[1:]
        ok = False
        for inv in cands:
            a = (pos32 * inv).astype(np.float32).astype(np.float64)
            if (np.abs(c[:, i] - np.cos(a)).max() <= one and
                    np.abs(s[:, i] - np.sin(a)).max() <= one):
                ok = True
                break
        assert ok, f"column {i}: no float32 angle pos * inv_freq reproduces the table"
    c64, s64 = O.rope_tables(max_seq, hd, theta)
    assert np.abs(c[4096:] - c64[4096:]).max() > 1e-5   # the two table builds differ
    assert np.abs(c[:8] - c64[:8]).max() < 1e-6


@pytest.mark.parametrize("hd,theta", [(64, 1e6), (128, 5e5)])
def test_rope_vs_complex_rotation(hd, theta):
    c, s = O.rope_tables(300, hd, theta)
    assert np.array_equal(c[0], np.ones(hd, np.float32)) and not s[0].any()
    half = hd // 2
    g = np.random.default_rng(hd)
    head = g.standard_normal(hd, dtype=np.float32)
    assert np.array_equal(O.rope_apply(head, c[0], s[0]), head)
    for pos in (1, 17, 299):
        out = O.rope_apply(head, c[pos], s[pos])
        freq = theta ** (-(2.0 * np.arange(half)) / hd)
        z = (head[:half] + 1j * head[half:]).astype(np.complex128) * np.exp(1j * pos * freq)
        assert np.allclose(out[:half], z.real, atol=2e-5) and np.allclose(out[half:], z.imag, atol=2e-5)
        assert np.allclose(np.hypot(out[:half], out[half:]), np.hypot(head[:half], head[half:]),
                           rtol=1e-5)


@pytest.mark.parametrize("hq,hkv,hd,seq", [(14, 2, 64, 300), (32, 8, 128, 97), (4, 4, 64, 2)])
def test_attention_vs_sdpa(hq, hkv, hd, seq):
    g = np.random.default_rng(seq)
    max_seq = seq + 5
    q = g.standard_normal((hq, hd), dtype=np.float32)
    kc = g.standard_normal((hkv, max_seq, hd), dtype=np.float32)
    vc = g.standard_normal((hkv, max_seq, hd), dtype=np.float32)
    out = O.attention(q, kc, vc, seq)
    T = lambda a: torch.from_numpy(a.astype(np.float64))
    ref = F.scaled_dot_product_attention(T(q)[None, :, None], T(kc[:, :seq])[None],
                                         T(vc[:, :seq])[None], enable_gqa=True)[0, :, 0].numpy()
    assert rel(out, ref) < 1e-5


@pytest.mark.parametrize("hq,hkv,hd,seq", [(14, 2, 64, 300), (32, 8, 128, 97), (4, 4, 64, 1)])
def test_attention_layer_vs_sdpa(hq, hkv, hd, seq):
    """The per-layer steps' attention (fused_ops.rs:823-858, 997-1040): no
    single-position shortcut, no clamp, out += w * v."""
    g = np.random.default_rng(seq + 1)
    max_seq = seq + 5
    q = g.standard_normal((hq, hd), dtype=np.float32)
    kc = g.standard_normal((hkv, max_seq, hd), dtype=np.float32)
    vc = g.standard_normal((hkv, max_seq, hd), dtype=np.float32)
    out = O.attention_layer(q, kc, vc, seq)
    T = lambda a: torch.from_numpy(a.astype(np.float64))
    ref = F.scaled_dot_product_attention(T(q)[None, :, None], T(kc[:, :seq])[None],
                                         T(vc[:, :seq])[None], enable_gqa=True)[0, :, 0].numpy()
    assert rel(out, ref) < 1e-5
    if seq == 1:
        assert np.array_equal(out, np.repeat(vc[:, 0], hq // hkv, 0))


def test_attention_native_cap_32768():
    """The native step scores only positions 0 .. min(seq_len, 32768) - 1
    (decoder.rs:1179-1184); the per-layer path scores them all.  Keys past
    32768 are made to dominate the scores, so an uncapped attention lands far
    from SDPA over the first 32768 keys and a capped one within 1e-5."""
    g = np.random.default_rng(32768)
    hq, hkv, hd, seq = 4, 2, 64, 32800
    q = g.standard_normal((hq, hd), dtype=np.float32) * np.float32(0.1)
    kc = g.standard_normal((hkv, seq, hd), dtype=np.float32)
    vc = g.standard_normal((hkv, seq, hd), dtype=np.float32)
    kc[:, 32768:] = np.repeat(q[::hq // hkv, None, :] * 200, seq - 32768, 1)   # huge scores
    vc[:, 32768:] = 1000.0
    T = lambda a: torch.from_numpy(a.astype(np.float64))

    def sdpa(n):
        return F.scaled_dot_product_attention(T(q)[None, :, None], T(kc[:, :n])[None],
                                              T(vc[:, :n])[None], enable_gqa=True)[0, :, 0].numpy()

    first = sdpa(32768)
    assert rel(O.attention(q, kc, vc, seq), first) < 1e-5
    assert rel(O.attention(q, kc, vc, 32768), first) < 1e-5
    whole = O.attention_layer(q, kc, vc, seq)
    assert rel(whole, sdpa(seq)) < 1e-5 and rel(whole, first) > 1.0


def test_attention_special_cases():
    g = np.random.default_rng(0)
    q = g.standard_normal((4, 64), dtype=np.float32)
    kc = g.standard_normal((2, 16, 64), dtype=np.float32)
    vc = g.standard_normal((2, 16, 64), dtype=np.float32)
    out = O.attention(q, kc, vc, 1)
    assert np.array_equal(out[:2], np.repeat(vc[0, :1], 2, 0))
    assert np.array_equal(out[2:], np.repeat(vc[1, :1], 2, 0))
    kc[:] = kc[:, :1]
    out = O.attention(q, kc, vc, 10)
    assert np.allclose(out[0], vc[0, :10].mean(0), atol=1e-6)


def test_argmax_kat_and_ties():
    lg = np.sin(np.arange(4096, dtype=np.float32) * np.float32(0.013)).astype(np.float32)
    lg[1234] = 100.0
    assert O.argmax(lg) == 1234
    lg = np.zeros(10, np.float32)
    lg[[3, 7]] = 5.0
    assert O.argmax(lg) == 3


# ------------------------------------------------------------ decoder step ---

def torch_step(w, cfg, kv, tok, pos, gs, f16=False, wkind=4, lmkind=4, tables=None, a8=False):
    """One decoder step in float64 from torch library ops (independent of the
    oracle's C code): rms_norm, RoPE, SDPA with GQA, silu.  f16: QKV, O, down
    and lm_head use binary16-rounded scales (numpy's float16), the effect of the
    reference's v2 repack at group 64 (decoder.rs:361-390).  wkind / lmkind: 4
    INT4 grouped, 8 INT8 per-row, 32 fp32.  tables: (cos, sin) [max_seq, hd] for a
    rotate-half RoPE (model.py:125-136); None = the exact complex rotation.
    a8: every INT4 projection contracts its input's bytes (u - 128) * s_x from
    the pinned quantize_act_u8 (the W4A8 step of a VNNI host at group 64)."""
    D = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    r16 = (lambda s: s.astype(np.float16).astype(np.float32)) if f16 else (lambda s: s)

    def A(v, kind=4):   # a projection input, byte-rounded under a8
        if not (a8 and kind == 4):
            return v
        u8, sx = O.quantize_act_u8(v.numpy().astype(np.float32))
        return D((u8.astype(np.float64) - 128) * sx)

    def deq(wt, sc, k, kind, f16s=False):
        if kind == 4:
            return D(dequant(wt, r16(sc) if f16s else sc, k, gs))
        if kind == 8:
            return D(wt.astype(np.float64) * np.asarray(sc, np.float64).reshape(-1, 1))
        return D(wt)

    H, hq, hkv, hd = cfg["hidden"], cfg["num_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    half = hd // 2
    if tables is None:
        freq = D(cfg["rope_theta"] ** (-(2.0 * np.arange(half)) / hd))
        rot = torch.exp(1j * pos * freq)

        def rope(t):   # [heads, hd]
            z = torch.complex(t[:, :half], t[:, half:]) * rot
            return torch.cat([z.real, z.imag], -1)
    else:
        cr, sr = D(tables[0][pos]), D(tables[1][pos])

        def rope(t):
            return t * cr + torch.cat([-t[:, half:], t[:, :half]], -1) * sr

    x = D(w["embed"][tok])
    for li, lw in enumerate(w["layers"]):
        xn = F.rms_norm(x, (H,), D(lw["in_norm"]), eps=cfg["eps"])
        qkv = deq(lw["qkv_w"], lw["qkv_s"], H, wkind, True) @ A(xn, wkind)
        if lw.get("qkv_b") is not None:
            qkv = qkv + D(lw["qkv_b"])
        q = rope(qkv[:hq * hd].reshape(hq, hd))
        k = rope(qkv[hq * hd:(hq + hkv) * hd].reshape(hkv, hd))
        v = qkv[(hq + hkv) * hd:].reshape(hkv, hd)
        kc, vc = kv[li]
        kc[:, pos] = k
        vc[:, pos] = v
        att = F.scaled_dot_product_attention(q[None, :, None], kc[None, :, :pos + 1],
                                             vc[None, :, :pos + 1], enable_gqa=True)[0, :, 0]
        x = x + deq(lw["o_w"], lw["o_s"], hq * hd, wkind, True) @ A(att.reshape(-1), wkind)
        xn = F.rms_norm(x, (H,), D(lw["post_norm"]), eps=cfg["eps"])
        h = F.silu(deq(lw["gate_w"], lw["gate_s"], H, wkind) @ A(xn, wkind)) * \
            (deq(lw["up_w"], lw["up_s"], H, wkind) @ A(xn, wkind))
        x = x + deq(lw["down_w"], lw["down_s"], cfg["intermediate"], wkind, True) @ A(h, wkind)
    xn = F.rms_norm(x, (H,), D(w["final_norm"]), eps=cfg["eps"])
    return (deq(w["lm_head_w"], w["lm_head_s"], H, lmkind, True) @ A(xn, lmkind)).numpy()


@pytest.mark.parametrize("gs,vocab,v2", [(32, 300, False), (64, 300, False), (64, 320, True)])
def test_decoder_step_vs_torch_float64(gs, vocab, v2):
    """v2: group 64 with every dimension a multiple of 64 (vocab 320) -> the
    reference's v2 repack (f16 scales on QKV / O / down / lm_head); vocab 300
    keeps the v1 f32 scales."""
    cfg = dict(num_layers=2, hidden=128, intermediate=256, num_heads=4, num_kv_heads=2,
               head_dim=32 * 2, vocab=vocab, eps=1e-6, rope_theta=1e6, qkv_bias=True)
    max_seq, pre = 24, 9
    w = synth.decoder_weights(cfg, 21, 4, 4, gs)
    ocfg = dict(num_layers=2, hidden=128, intermediate=256, num_heads=4, num_kv_heads=2,
                head_dim=64, vocab=vocab, group_size=gs, max_seq=max_seq, rope_theta=1e6,
                eps=1e-6, wkind=4, lmkind=4)
    dec = O.Decoder(w, ocfg)
    kvp = synth.kv_prefill(cfg, 21, pre, max_seq)
    tkv = []
    for li, (k, v) in enumerate(kvp):
        dec.copy_kv(li, k, v, pre)
        tkv.append((torch.from_numpy(k.astype(np.float64)), torch.from_numpy(v.astype(np.float64))))
    tok = 17
    for step in range(4):
        pos = pre + step
        lo = dec.step(tok, pos)
        kv_other = [(k.clone(), v.clone()) for k, v in tkv]
        lt = torch_step(w, cfg, tkv, tok, pos, gs, f16=v2)
        assert rel(lo, lt) < 1e-5, f"step {step}"
        if gs == 64:   # the scale precision is visible: the other model is off by > 1e-4
            assert rel(lo, torch_step(w, cfg, kv_other, tok, pos, gs, f16=not v2)) > 1e-4
        assert O.argmax(lo) == int(np.argmax(lt))
        tok = O.argmax(lo)
    assert dec.kv_len() == pre + 4
    # out-of-range token / position -> zeroed logits (decoder.rs:1066-1089)
    assert not dec.step(vocab, 3).any() and not dec.step(1, max_seq).any()
    dec.close()


@pytest.mark.parametrize("vocab,v2", [(300, False), (320, True)])
def test_decoder_step_a8_vs_torch_float64(vocab, v2):
    """The W4A8 step of a VNNI host at group 64 (orc_decoder_set_a8): every INT4
    projection input byte-rounded (the SwiGLU pair, decoder.rs:1262-1282; QKV,
    O, down and the lm_head through projection_gemv, decoder.rs:1029-1049).
    Against the float64 model on the same byte rounding (measured 1e-7; the
    bar leaves room for an occasional rounding flip); the exact W4A32 step is
    off by 2-4%."""
    cfg = dict(num_layers=2, hidden=128, intermediate=256, num_heads=4, num_kv_heads=2,
               head_dim=64, vocab=vocab, eps=1e-6, rope_theta=1e6, qkv_bias=True)
    max_seq, pre, gs = 24, 9, 64
    w = synth.decoder_weights(cfg, 23, 4, 4, gs)
    ocfg = dict(num_layers=2, hidden=128, intermediate=256, num_heads=4, num_kv_heads=2,
                head_dim=64, vocab=vocab, group_size=gs, max_seq=max_seq, rope_theta=1e6,
                eps=1e-6, wkind=4, lmkind=4)
    dec, exact = O.Decoder(w, ocfg, a8=True), O.Decoder(w, ocfg)
    kvp = synth.kv_prefill(cfg, 23, pre, max_seq)
    tkv = []
    for li, (k, v) in enumerate(kvp):
        dec.copy_kv(li, k, v, pre)
        exact.copy_kv(li, k, v, pre)
        tkv.append((torch.from_numpy(k.astype(np.float64)), torch.from_numpy(v.astype(np.float64))))
    tok = 5
    for step in range(4):
        pos = pre + step
        lo = dec.step(tok, pos)
        lt = torch_step(w, cfg, tkv, tok, pos, gs, f16=v2, a8=True)
        assert rel(lo, lt) < 1e-4, f"step {step}"
        assert rel(lo, exact.step(tok, pos)) > 1e-2
        tok = O.argmax(lo)
    dec.close()
    exact.close()


@pytest.mark.parametrize("wkind,lmkind,layer_path", [(4, 32, True), (8, 8, True), (8, 32, False),
                                                      (4, 8, False), (4, 4, True)])
def test_decoder_kinds_and_layer_path_vs_torch_float64(wkind, lmkind, layer_path):
    """INT8 projections and INT8 / fp32 lm_heads (configs 4 and 5-INT8), with the
    per-layer path's f32 RoPE tables passed in and its numerics
    (orc_decoder_set_layer_path), against the float64 torch model using the
    same tables; a model with the exact rotation is visibly different once the
    position is in the thousands."""
    from torchburn_amd.decoder import rotary_tables_f32
    cfg = dict(num_layers=2, hidden=128, intermediate=256, num_heads=4, num_kv_heads=2,
               head_dim=64, vocab=300, eps=1e-5, rope_theta=5e5, qkv_bias=wkind == 4)
    max_seq, pre = 3010, 3000
    w = synth.decoder_weights(cfg, 31 + wkind + lmkind, wkind, lmkind, 32)
    ocfg = dict(cfg, group_size=32, max_seq=max_seq, wkind=wkind, lmkind=lmkind)
    tabs = rotary_tables_f32(max_seq, 64, 5e5)
    dec = O.Decoder(w, ocfg, rope_tables=tabs, layer_path=layer_path)
    kvp = synth.kv_prefill(cfg, 5, pre, max_seq)
    tkv = []
    for li, (k, v) in enumerate(kvp):
        dec.copy_kv(li, k, v, pre)
        tkv.append((torch.from_numpy(k.astype(np.float64)), torch.from_numpy(v.astype(np.float64))))
    tok = 17
    for step in range(3):
        pos = pre + step
        lo = dec.step(tok, pos)
        exact = [(k.clone(), v.clone()) for k, v in tkv]
        lt = torch_step(w, cfg, tkv, tok, pos, 32, wkind=wkind, lmkind=lmkind, tables=tabs)
        assert rel(lo, lt) < 1e-5, f"step {step}"
        if step == 0:
            le = torch_step(w, cfg, exact, tok, pos, 32, wkind=wkind, lmkind=lmkind)
            assert rel(lt, le) > 1e-5
        assert O.argmax(lo) == int(np.argmax(lt))
        tok = O.argmax(lo)
    dec.close()

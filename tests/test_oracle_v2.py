"""Pins the oracle's v2-layout and W4A8 restatements (oracle/tb_oracle.c, f2).

  f16 decode      all 65536 bit patterns against numpy's float16 -> float32
  f16 encode      numpy's float32 -> float16 (IEEE round to nearest even) on every
                  f16 rounding boundary, its neighbours and random bit patterns;
                  NaN -> sign | 0x7E00 and overflow -> inf as packed_v2.rs:66-105;
                  the reference's round-trip values (packed_v2.rs:713-740)
  v1 -> v2 pack   the reference's LCG case (packed_v2.rs:742-771): nibble bytes
                  identical, scale bytes = numpy float16 bits
  v2 GEMV         bit-identical to the v1 g64 GEMV run on the f16-rounded scales
                  (same lane restatement, a different code path through the
                  blocks); the reference's v2-vs-v1 budgets (int4.rs:260-300,
                  packed_v2.rs:773-820)
  W4A8 quantize   closed forms: the max element maps to +-127, exact multiples of
                  s_x map to their integer, ties round to even, zero input
  W4A8 GEMV       float64 integer brute force; equal to the exact W4A32 result
                  when x is already on the s_x grid; v1 and v2 forms agree
"""
import numpy as np
import pytest

from oracle import oracle as O


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-6))


# ------------------------------------------------------------------- f16 ---

def test_f16_decode_all_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_bits_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _boundary_values():
    """Every f16 value, the midpoints between neighbours (ties) and one f32 ulp
    either side of each midpoint, for both signs."""
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)
    v = h.view(np.float16).astype(np.float64)
    nxt = np.append(v[1:], 65520.0)            # 65520 = overflow threshold
    mid = ((v + nxt) / 2).astype(np.float32)
    up = np.nextafter(mid, np.float32(np.inf))
    dn = np.nextafter(mid, np.float32(0))
    pos = np.concatenate([v.astype(np.float32), mid, up, dn,
                          np.float32([65504, 65519.996, 65520, 1e6, 3e38, 2.0 ** -25,
                                      2.0 ** -26, 1e-10, 5.96e-8])])
    return np.concatenate([pos, -pos]).astype(np.float32)


def test_f16_encode_matches_ieee_rne():
    vals = _boundary_values()
    rng = np.random.default_rng(5)
    rand = rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    vals = np.concatenate([vals, rand[~np.isnan(rand)]])
    got = O.f32_to_f16_bits(vals)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f16_encode_nan_and_inf():
    vals = np.float32([np.nan, -np.nan, np.inf, -np.inf])
    vals[1] = -np.abs(vals[1])
    got = O.f32_to_f16_bits(vals)
    assert list(got) == [0x7E00, 0xFE00, 0x7C00, 0xFC00]


def test_f16_round_trip_reference_values():
    # packed_v2.rs:713-740
    for v in [0.0, -0.0, 1.0, -1.0, 0.5, 2.0, 65504.0, -3.75, 1234.5, 1e-4, 6.0e-5, 6.1e-8]:
        back = O.f16_bits_to_f32(O.f32_to_f16_bits(np.float32([v])))[0]
        if v == 0.0:
            assert back == 0.0 and np.signbit(back) == np.signbit(v)
        elif abs(v) < 6.1e-5:
            assert abs(back - v) < 6e-8
        else:
            assert abs((back - v) / v) < 6e-4
    big = O.f16_bits_to_f32(O.f32_to_f16_bits(np.float32([1e6, -1e6])))
    assert big[0] == np.inf and big[1] == -np.inf


# ------------------------------------------------------------- v2 packing ---

def _lcg(seed):
    while True:
        seed = (seed * 6364136223846793005 + 1442695040888963407) % 2 ** 64
        yield seed >> 33


def test_pack_v1_to_v2_reference_case():
    # packed_v2.rs:742-771: n = 3, k = 128, LCG seed 42, scales 0.01 + 0.001 i
    n, k = 3, 128
    g = _lcg(42)
    src = np.array([next(g) & 0xFF for _ in range(n * k // 2)], np.uint8).reshape(n, k // 2)
    sc = (0.01 + np.arange(n * 2, dtype=np.float32) * np.float32(0.001)).astype(np.float32)
    sc = sc.reshape(n, 2)
    out = O.pack_v1_to_v2(src, sc, k)
    assert out.shape == (n, 2 * 34)
    blk = out.reshape(n, 2, 34)
    assert np.array_equal(blk[:, :, :32], src.reshape(n, 2, 32))
    bits = blk[:, :, 32].astype(np.uint16) | (blk[:, :, 33].astype(np.uint16) << 8)
    assert np.array_equal(bits, sc.astype(np.float16).view(np.uint16))
    back = bits.view(np.float16).astype(np.float32)
    assert (np.abs(back - sc) / sc).max() < 6e-4


def _f16_round(s):
    return s.astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("m,n,k", [(1, 64, 896), (3, 37, 128), (2, 200, 4096)])
def test_gemv_v2_equals_v1_on_f16_scales(m, n, k):
    rng = np.random.default_rng(n + k)
    w = rng.standard_normal((n, k)).astype(np.float32)
    wq, sc = O.quantize_int4_grouped(w, 64)
    x = rng.standard_normal((m, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    v2 = O.gemm_w4_v2(x, O.pack_v1_to_v2(wq, sc, k), bias)
    v1 = O.gemm_w4(x, wq, _f16_round(sc), bias, group_size=64)
    assert np.array_equal(v2.view(np.uint32), v1.view(np.uint32))
    # and within the f16-scale budget of the f32-scale v1 result (int4.rs:291-299)
    assert rel(v2, O.gemm_w4(x, wq, sc, bias, group_size=64)) < 5e-3


def test_gemv_v2_reference_cases():
    # int4.rs:260-300: n 64, k 896, x = sin(0.19 i) * 2, w = cos(0.31 i) * 1.5
    n, k = 64, 896
    x = (np.sin(np.arange(k, dtype=np.float32) * np.float32(0.19)) * 2).astype(np.float32)
    w = (np.cos(np.arange(n * k, dtype=np.float32) * np.float32(0.31)) * 1.5).astype(np.float32)
    wq, sc = O.quantize_int4_grouped(w.reshape(n, k), 64)
    v2 = O.gemm_w4_v2(x.reshape(1, k), O.pack_v1_to_v2(wq, sc, k))
    assert rel(v2, O.gemm_w4(x.reshape(1, k), wq, sc, group_size=64)) < 5e-3
    # packed_v2.rs:773-820: n 8, k 128, LCG seed 7; |v1 - v2| < 5e-3 max(|v1|, 1)
    n, k = 8, 128
    g = _lcg(7)
    wb = np.array([next(g) & 0xFF for _ in range(n * k // 2)], np.uint8).reshape(n, k // 2)
    s = np.array([0.002 + (next(g) % 1000) * 1e-5 for _ in range(n * 2)], np.float32)
    s = s.reshape(n, 2)
    xs = np.array([((next(g) % 2000) - 1000.0) / 500.0 for _ in range(k)], np.float32)
    a = O.gemm_w4(xs.reshape(1, k), wb, s, group_size=64)[0]
    b = O.gemm_w4_v2(xs.reshape(1, k), O.pack_v1_to_v2(wb, s, k))[0]
    assert np.all(np.abs(a - b) < 5e-3 * np.maximum(np.abs(a), 1.0))


# ------------------------------------------------------------------ W4A8 ---

def test_quantize_act_closed_forms():
    # s_x = 127 / 127 = 1 exactly: x on the integer grid maps to itself.  The
    # first 16 * (k / 16) elements round ties to even (cvtps_epi32), the tail
    # rounds them away from zero (f32::round, gemv.rs:1383-1386).
    vals = [127.0, -127.0, 0.0, 2.5, 3.5, -2.5, 1.49, 100.0]
    x = np.float32(vals + vals + vals[:4] + [2.5, -2.5, 0.5, -0.5])   # k = 24: 16 + 8 tail
    u, sx = O.quantize_act_u8(x)
    assert sx == 1.0
    body = [127, -127, 0, 2, 4, -2, 1, 100]
    assert list(u.astype(int) - 128) == body + body + [127, -127, 0, 3, 3, -3, 1, -1]
    u8, _ = O.quantize_act_u8(np.float32(vals))   # k = 8: all tail
    assert list(u8.astype(int) - 128) == [127, -127, 0, 3, 4, -3, 1, 100]
    un, _ = O.quantize_act_u8(np.float32([np.nan] + (vals + vals)[:15] + [np.nan, 1.0]))
    assert un[0] == 128 and un[16] == 128
    # the largest |x| maps to +-127 whatever its scale
    rng = np.random.default_rng(1)
    for _ in range(20):
        x = rng.standard_normal(256).astype(np.float32) * np.float32(10 ** rng.uniform(-6, 6))
        u, sx = O.quantize_act_u8(x)
        i = int(np.abs(x).argmax())
        assert int(u[i]) - 128 == (127 if x[i] > 0 else -127)
        assert np.all((u >= 1) & (u <= 255))
        assert sx == np.float32(np.abs(x).max()) / np.float32(127.0)
    u, sx = O.quantize_act_u8(np.zeros(64, np.float32))
    assert np.all(u == 128) and sx == np.float32(1e-10) / np.float32(127.0)


@pytest.mark.parametrize("n,k", [(16, 64), (64, 896), (37, 4096)])
def test_w4a8_gemv(n, k):
    rng = np.random.default_rng(k)
    wq, sc = O.quantize_int4_grouped(rng.standard_normal((n, k)).astype(np.float32), 64)
    x = rng.standard_normal((2, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    y = O.gemm_w4a8_g64(x, wq, sc, bias)
    q = O.unpack_int4(wq, k).astype(np.float64)
    for i in range(2):
        u, sx = O.quantize_act_u8(x[i])
        xi = u.astype(np.float64) - 128
        grp = (q * xi).reshape(n, k // 64, 64).sum(-1)          # exact integers
        want = (grp * (np.float64(sx) * sc.astype(np.float64))).sum(-1) + bias
        assert rel(y[i], want) < 1e-6
    # v2 blocks carry f16 scales: the blocked form equals the v1 form on them
    yb = O.gemm_w4a8_g64(x, O.pack_v1_to_v2(wq, sc, k), None, bias, blocked=True)
    y16 = O.gemm_w4a8_g64(x, wq, _f16_round(sc), bias)
    assert np.array_equal(yb.view(np.uint32), y16.view(np.uint32))


@pytest.mark.parametrize("n,k", [(24, 1000), (9, 20504)])
def test_w4a8_gemv_short_last_group(n, k):
    """K % 64 != 0 (and K % 16 != 0 for 1000): the reference's VNNI row reads its
    last group past the row (undefined); the oracle counts the missing elements
    as zero.  Float64 over exact integer group sums, with the activation bytes
    from the quantizer pinned above."""
    rng = np.random.default_rng(k)
    ng = (k + 63) // 64
    nib = rng.integers(0, 16, (n, k)).astype(np.uint8)
    wq = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    sc = (np.abs(rng.normal(0, 0.02, (n, ng))) + 1e-3).astype(np.float32)
    x = rng.standard_normal((2, k)).astype(np.float32)
    y = O.gemm_w4a8_g64(x, wq, sc)
    q = nib.astype(np.float64) - 8
    for i in range(2):
        u, sx = O.quantize_act_u8(x[i])
        prod = q * (u.astype(np.float64) - 128)
        pad = np.zeros((n, ng * 64))
        pad[:, :k] = prod
        grp = pad.reshape(n, ng, 64).sum(-1)
        want = (grp * (np.float64(sx) * sc.astype(np.float64))).sum(-1)
        assert rel(y[i], want) < 1e-6


def test_w4a8_equals_w4a32_on_the_grid():
    """x already on the s_x grid (integers with max 127 -> s_x = 1): the u8
    quantization is lossless and W4A8 equals the exact W4A32 contraction."""
    rng = np.random.default_rng(3)
    n, k = 48, 512
    wq, sc = O.quantize_int4_grouped(rng.standard_normal((n, k)).astype(np.float32), 64)
    x = rng.integers(-127, 128, (1, k)).astype(np.float32)
    x[0, 5] = 127.0
    y8 = O.gemm_w4a8_g64(x, wq, sc)
    y32 = O.gemv_w4_f64(x[0], wq, sc, group_size=64)
    assert rel(y8[0], y32) < 1e-6


def test_swiglu_mlp_w4a8_composition():
    """The W4A8 fused MLP (fused_ops.rs:215-232, 409-421) is the pinned W4A8 GEMV
    composed: h = silu(g + gb) * (u + ub) over the gate and up GEMVs on x's
    bytes, then the down GEMV on h's bytes with its bias.  A float64 model with
    the same byte rounding lands within the few-quantum slack of rounding h."""
    rng = np.random.default_rng(77)
    m, k, inter, nout = 2, 512, 192, 320
    gw, gsc = O.quantize_int4_grouped(rng.standard_normal((inter, k)).astype(np.float32), 64)
    uw, usc = O.quantize_int4_grouped(rng.standard_normal((inter, k)).astype(np.float32), 64)
    dw, dsc = O.quantize_int4_grouped(rng.standard_normal((nout, inter)).astype(np.float32), 64)
    gb, ub, db = (rng.standard_normal(n).astype(np.float32) for n in (inter, inter, nout))
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = O.swiglu_mlp_w4a8(x, gw, gsc, uw, usc, dw, dsc, gb, ub, db)
    g = O.gemm_w4a8_g64(x, gw, gsc) + gb
    u = O.gemm_w4a8_g64(x, uw, usc) + ub
    h = (g / (np.float32(1) + np.exp(-g)) * u).astype(np.float32)
    assert rel(y, O.gemm_w4a8_g64(h, dw, dsc, db)) < 1e-6
    # float64: exact integer group sums of the bytes, f64 SwiGLU, then h's bytes
    q = lambda w_, n_, kk: O.unpack_int4(w_, kk).astype(np.float64).reshape(n_, kk // 64, 64)
    def a8(v, w_, s_, n_, kk):
        u8, sx = O.quantize_act_u8(v)
        xi = (u8.astype(np.float64) - 128).reshape(kk // 64, 64)
        return ((q(w_, n_, kk) * xi).sum(-1) * (np.float64(sx) * s_.astype(np.float64))).sum(-1)
    for i in range(m):
        g64 = a8(x[i], gw, gsc, inter, k) + gb
        u64 = a8(x[i], uw, usc, inter, k) + ub
        h64 = g64 / (1 + np.exp(-g64)) * u64
        want = a8(h64.astype(np.float32), dw, dsc, nout, inter) + db
        assert rel(y[i], want) < 2e-3
    y32 = O.swiglu_mlp_w4(x, gw, gsc, uw, usc, dw, dsc, gb, ub, db, group_size=64)
    assert rel(y, y32) > 1e-2

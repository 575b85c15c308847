/*
 * tb_oracle.c -- CPU restatement of TorchBurn's quantized decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP kernels in
 * torchburn_amd/csrc are compared against, and the CPU baseline that bench.py
 * times beside the GPU.  Nothing in the product path may call it.
 *
 * Every function restates the algorithm of the Rust reference at
 * /root/reference (kuntal-devrat/torchburn), cited as file:line.  The SIMD
 * kernels of the reference are restated lane by lane in plain C: a 16-float
 * array stands for one __m512 register, fmaf() for _mm512_fmadd_ps (single
 * rounding), and tree16() for _mm512_reduce_add_ps.  The file is built with
 * -ffp-contract=off so that every "a * b + c" that the reference writes as two
 * operations stays two operations.
 *
 * Hot loops carry target_clones so one .so runs on AVX-512, AVX2 or plain
 * x86-64 hosts (the GPU box's CPU is not this container's CPU).
 *
 * Parity status of each function is listed in the header of tests/test_oracle.py
 * (what pins it) -- every function here has at least one pinning check.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))
#define HOT __attribute__((target_clones("avx512f", "avx2", "default")))

enum { L16 = 16 };

/* Rayon's minimum task length for row loops, gemv.rs:1535-1536:           */
/* max(N / (4 * threads), 8).  Only scheduling -- no cross-row reduction.   */
static int64_t rayon_chunk(int64_t n) {
#ifdef _OPENMP
    int64_t t = omp_get_max_threads();
#else
    int64_t t = 1;
#endif
    int64_t c = n / (4 * t);
    return c > 8 ? c : 8;
}

/* _mm512_reduce_add_ps: halves added pairwise, 512 -> 256 -> 128 -> 64 -> 32.
 * The exact order is LLVM's and is not pinned at the bit level (see the
 * tolerance-based tests); this is the natural tree. */
static inline float tree16(const float *a) {
    float t8[8], t4[4];
    for (int i = 0; i < 8; ++i) t8[i] = a[i] + a[i + 8];
    for (int i = 0; i < 4; ++i) t4[i] = t8[i] + t8[i + 4];
    float t0 = t4[0] + t4[2], t1 = t4[1] + t4[3];
    return t0 + t1;
}

/* ------------------------------------------------------------------------ */
/* a1: INT4 v1 packing.  python/torchburn/quantization.py:89-94 packs          */
/*   byte[n, j] = (q[n,2j] + 8) | ((q[n,2j+1] + 8) << 4),  q in [-8, 7];      */
/* unpack (gemv.rs:1486-1502) is nib - 8.  Odd K: the last byte's high nibble */
/* is element K which does not exist; it is written as 0 (q = -8 is never     */
/* read back).                                                                */
/* ------------------------------------------------------------------------ */
ORC_API void orc_pack_int4(const int8_t *q, uint8_t *out, int64_t n, int64_t k) {
    int64_t bpr = (k + 1) / 2;
    for (int64_t r = 0; r < n; ++r) {
        const int8_t *qr = q + r * k;
        uint8_t *o = out + r * bpr;
        for (int64_t j = 0; j < bpr; ++j) {
            uint8_t lo = (uint8_t)((qr[2 * j] + 8) & 0x0F);
            uint8_t hi = (2 * j + 1 < k) ? (uint8_t)((qr[2 * j + 1] + 8) & 0x0F) : 0;
            o[j] = (uint8_t)(lo | (hi << 4));
        }
    }
}

ORC_API void orc_unpack_int4(const uint8_t *w, int8_t *q, int64_t n, int64_t k) {
    int64_t bpr = (k + 1) / 2;
    for (int64_t r = 0; r < n; ++r)
        for (int64_t i = 0; i < k; ++i) {
            uint8_t b = w[r * bpr + i / 2];
            q[r * k + i] = (int8_t)(((i & 1) ? (b >> 4) : (b & 0x0F)) - 8);
        }
}

/* Grouped quantizer, quantization.py:53-118: s = max(amax/7, 1e-8) per group, */
/* q = clamp(round_half_even(w / s), -8, 7).  nearbyintf rounds half to even  */
/* in the default rounding mode, as torch.round does.                         */
ORC_API void orc_quantize_int4_grouped(const float *w, uint8_t *packed, float *scales,
                                       int64_t n, int64_t k, int64_t gs) {
    int64_t ng = k / gs, bpr = (k + 1) / 2;
    int8_t *q = (int8_t *)malloc((size_t)k);
    for (int64_t r = 0; r < n; ++r) {
        for (int64_t g = 0; g < ng; ++g) {
            float amax = 0.f;
            for (int64_t i = 0; i < gs; ++i) {
                float a = fabsf(w[r * k + g * gs + i]);
                amax = a > amax ? a : amax;
            }
            float s = amax / 7.0f;
            if (s < 1e-8f) s = 1e-8f;
            scales[r * ng + g] = s;
            for (int64_t i = 0; i < gs; ++i) {
                float v = nearbyintf(w[r * k + g * gs + i] / s);
                v = v < -8.f ? -8.f : (v > 7.f ? 7.f : v);
                q[g * gs + i] = (int8_t)v;
            }
        }
        orc_pack_int4(q, packed + r * bpr, 1, k);
    }
    free(q);
}

/* ------------------------------------------------------------------------ */
/* a2: scalar exact group dot, gemv.rs:1486-1502 (sequential f32 sum).        */
/* ------------------------------------------------------------------------ */
static float dot_u4_group_scalar(const float *x, const uint8_t *w, int64_t len) {
    float t = 0.f;
    for (int64_t i = 0; i < len; ++i) {
        uint8_t b = w[i / 2];
        int q = ((i & 1) ? (b >> 4) : (b & 0x0F)) - 8;
        t += x[i] * (float)q;
    }
    return t;
}

/* a3: unpack_and_fma_32_avx512, gemv.rs:1190-1211.  16 bytes -> elements     */
/* 0..15 (lane i) and 16..31 (lane i); result lane i = fma(w1, x1, w0 * x0).   */
static inline void unpack_fma32(const float *x, const uint8_t *w, float *out16) {
    float q[32];
    for (int j = 0; j < 16; ++j) {   /* element 2j: low nibble, 2j+1: high nibble */
        q[2 * j] = (float)((int)(w[j] & 0x0F) - 8);
        q[2 * j + 1] = (float)((int)(w[j] >> 4) - 8);
    }
    for (int i = 0; i < L16; ++i) {
        float m0 = q[i] * x[i];
        out16[i] = fmaf(q[16 + i], x[16 + i], m0);
    }
}

/* a4: one output row.  group 32: gemv.rs:1279-1299; group 64: 1253-1275;     */
/* other group sizes: the scalar per-group fallback at gemv.rs:1650-1660.     */
static inline float w4_row(const float *x, const uint8_t *wr, const float *sr, int64_t k,
                           int64_t gs) {
    int64_t ng = (k + gs - 1) / gs;
    if ((gs == 32 || gs == 64) && k % gs == 0) {
        float acc[L16] = {0}, p0[L16], p1[L16];
        for (int64_t g = 0; g < ng; ++g) {
            float s = sr[g];
            if (gs == 32) {
                unpack_fma32(x + g * 32, wr + g * 16, p0);
                for (int i = 0; i < L16; ++i) acc[i] = fmaf(p0[i], s, acc[i]);
            } else {
                unpack_fma32(x + g * 64, wr + g * 32, p0);
                unpack_fma32(x + g * 64 + 32, wr + g * 32 + 16, p1);
                for (int i = 0; i < L16; ++i) acc[i] = fmaf(p0[i] + p1[i], s, acc[i]);
            }
        }
        return tree16(acc);
    }
    float t = 0.f;
    for (int64_t g = 0; g < ng; ++g) {
        int64_t len = (k - g * gs) < gs ? (k - g * gs) : gs;
        t += dot_u4_group_scalar(x + g * gs, wr + g * (gs / 2), len) * sr[g];
    }
    return t;
}

/* a5: gemv_w4a32_grouped, gemv.rs:1514-1684.  One task per output row       */
/* (Rayon par_iter, min chunk max(N/(4T), 8)); no cross-row reduction.        */
HOT static void w4_rows(const float *x, const uint8_t *w, const float *s, const float *bias,
                        float *y, int64_t r0, int64_t r1, int64_t k, int64_t gs) {
    int64_t ng = (k + gs - 1) / gs, bpr = (k + 1) / 2;
    for (int64_t r = r0; r < r1; ++r) {
        float v = w4_row(x, w + r * bpr, s + r * ng, k, gs);
        y[r] = v + (bias ? bias[r] : 0.f);
    }
}

ORC_API void orc_gemv_w4(const float *x, const uint8_t *w, const float *s, const float *bias,
                         float *y, int64_t n, int64_t k, int64_t gs) {
    int64_t ch = rayon_chunk(n);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t c = 0; c < (n + ch - 1) / ch; ++c)
        w4_rows(x, w, s, bias, y, c * ch, (c + 1) * ch < n ? (c + 1) * ch : n, k, gs);
}

/* a6: gemm_w4a32_grouped, gemv.rs:1690-1725: M independent GEMVs.          */
ORC_API void orc_gemm_w4(const float *x, const uint8_t *w, const float *s, const float *bias,
                         float *y, int64_t m, int64_t n, int64_t k, int64_t gs) {
    for (int64_t i = 0; i < m; ++i) orc_gemv_w4(x + i * k, w, s, bias, y + i * n, n, k, gs);
}

/* Float64 brute force of the same contraction (the "exact dequant-dot" of   */
/* tests/parity/int4.rs:109-126), used to pin the lane restatement above.     */
ORC_API void orc_gemv_w4_f64(const float *x, const uint8_t *w, const float *s,
                             const float *bias, double *y, int64_t n, int64_t k, int64_t gs) {
    int64_t ng = (k + gs - 1) / gs, bpr = (k + 1) / 2;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; ++r) {
        double t = 0.0;
        for (int64_t g = 0; g < ng; ++g) {
            double p = 0.0;
            for (int64_t i = g * gs; i < k && i < (g + 1) * gs; ++i) {
                uint8_t b = w[r * bpr + i / 2];
                int q = ((i & 1) ? (b >> 4) : (b & 0x0F)) - 8;
                p += (double)q * (double)x[i];
            }
            t += p * (double)s[r * ng + g];
        }
        y[r] = t + (bias ? (double)bias[r] : 0.0);
    }
}

/* ------------------------------------------------------------------------ */
/* f2: the v2 layout, packed_v2.rs:26-143.  One 34-byte block per 64-element  */
/* group: 32 bytes of v1 nibbles, then the group scale as IEEE binary16,       */
/* little-endian.                                                             */
/* ------------------------------------------------------------------------ */

/* binary16 -> binary32 (packed_v2.rs:32-56): exact for every finite value;   */
/* +-inf kept; any NaN becomes the default quiet NaN.                          */
ORC_API float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u;
    float v;
    if (e == 0)
        v = ldexpf((float)m, -24); /* zero or subnormal: m * 2^-24 */
    else if (e == 31)
        v = m ? NAN : INFINITY;
    else {
        uint32_t b = ((e + 112u) << 23) | (m << 13);
        memcpy(&v, &b, 4);
    }
    uint32_t bits;
    memcpy(&bits, &v, 4);
    if (!(e == 31 && m)) bits |= sign;
    memcpy(&v, &bits, 4);
    return v;
}

/* binary32 -> binary16, round to nearest even (packed_v2.rs:66-105):        */
/* overflow to +-inf, NaN to sign | 0x7E00, underflow to signed zero, with   */
/* RNE on the bits shifted out in the subnormal range.                        */
ORC_API uint16_t orc_f32_to_f16(float v) {
    uint32_t x;
    memcpy(&x, &v, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    int32_t e = (int32_t)((x >> 23) & 0xFFu);
    uint32_t m = x & 0x7FFFFFu;
    if (e == 0xFF) return sign | (m ? 0x7E00u : 0x7C00u);
    int32_t ub = e - 127;                  /* unbiased exponent */
    if (ub > 15) return sign | 0x7C00u;
    uint32_t sig, drop;                    /* significand and bits to drop */
    uint32_t base;
    if (ub >= -14) {                       /* normal half: keep 10 mantissa bits */
        sig = m;
        drop = 13;
        base = (uint32_t)(ub + 15) << 10;
    } else {
        if (ub < -25) return sign;          /* below half the smallest subnormal */
        sig = m | 0x800000u;                /* subnormal half: value = sig * 2^(ub-23) */
        drop = (uint32_t)(-ub - 1);         /* 14..24 bits */
        base = 0;
    }
    uint32_t keep = sig >> drop, rem = sig & ((1u << drop) - 1u), half = 1u << (drop - 1);
    uint32_t r = base + keep;             /* a carry may reach the exponent: still RNE */
    if (rem > half || (rem == half && (keep & 1u))) r += 1u;
    return sign | (uint16_t)r;
}

ORC_API void orc_f32_to_f16_n(const float *v, uint16_t *h, int64_t n) {
    for (int64_t i = 0; i < n; ++i) h[i] = orc_f32_to_f16(v[i]);
}

ORC_API void orc_f16_to_f32_n(const uint16_t *h, float *v, int64_t n) {
    for (int64_t i = 0; i < n; ++i) v[i] = orc_f16_to_f32(h[i]);
}

/* pack_rows_w4a32_group64_v1_to_v2, packed_v2.rs:114-143 (k % 64 == 0). */
ORC_API void orc_pack_v1_to_v2(const uint8_t *w, const float *s, uint8_t *out, int64_t n,
                               int64_t k) {
    int64_t ng = k / 64, bpr = k / 2;
    for (int64_t r = 0; r < n; ++r)
        for (int64_t g = 0; g < ng; ++g) {
            uint8_t *blk = out + (r * ng + g) * 34;
            memcpy(blk, w + r * bpr + g * 32, 32);
            uint16_t h = orc_f32_to_f16(s[r * ng + g]);
            blk[32] = (uint8_t)(h & 0xFF);
            blk[33] = (uint8_t)(h >> 8);
        }
}

static inline float v2_scale(const uint8_t *blk) {
    return orc_f16_to_f32((uint16_t)(blk[32] | (blk[33] << 8)));
}

/* v2 GEMV, exact tiers (packed_v2.rs:145-200, 326-485 without VNNI): per     */
/* group the two 32-element halves (unpack_fma32 on bytes 0..15 and 16..31),  */
/* added lane by lane, then acc = fma(sum, f16 scale, acc); tree16 at the end. */
HOT static void w4_v2_rows(const float *x, const uint8_t *w, const float *bias, float *y,
                           int64_t r0, int64_t r1, int64_t k) {
    int64_t ng = k / 64;
    for (int64_t r = r0; r < r1; ++r) {
        const uint8_t *wr = w + r * ng * 34;
        float acc[L16] = {0}, p0[L16], p1[L16];
        for (int64_t g = 0; g < ng; ++g) {
            const uint8_t *blk = wr + g * 34;
            float sc = v2_scale(blk);
            unpack_fma32(x + g * 64, blk, p0);
            unpack_fma32(x + g * 64 + 32, blk + 16, p1);
            for (int i = 0; i < L16; ++i) acc[i] = fmaf(p0[i] + p1[i], sc, acc[i]);
        }
        y[r] = tree16(acc) + (bias ? bias[r] : 0.f);
    }
}

ORC_API void orc_gemv_w4_v2(const float *x, const uint8_t *w, const float *bias, float *y,
                            int64_t n, int64_t k) {
    int64_t ch = rayon_chunk(n);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t c = 0; c < (n + ch - 1) / ch; ++c)
        w4_v2_rows(x, w, bias, y, c * ch, (c + 1) * ch < n ? (c + 1) * ch : n, k);
}

/* w4a32_grouped_linear_v2 for M rows (packed_v2.rs:541-550): M GEMVs. */
ORC_API void orc_gemm_w4_v2(const float *x, const uint8_t *w, const float *bias, float *y,
                            int64_t m, int64_t n, int64_t k) {
    for (int64_t i = 0; i < m; ++i) orc_gemv_w4_v2(x + i * k, w, bias, y + i * n, n, k);
}

/* ------------------------------------------------------------------------ */
/* f2: the W4A8 semantics of the AVX-512 VNNI tier at group 64.              */
/* quantize_activation_to_u8_avx512, gemv.rs:1353-1389: s_x = max(max|x|,   */
/* 1e-10) / 127; the first 16 * (k / 16) elements: q = round-to-nearest-even  */
/* (x * (1 / s_x)) (cvtps_epi32 under the default MXCSR), the rest (the       */
/* scalar tail, gemv.rs:1383-1386): q = round-half-away(x / s_x) clamped to   */
/* +-127; byte = q + 128.  NaN gives q = 0 either way (cvtps_epi32's integer  */
/* indefinite + 128 truncated to a byte; Rust's NaN as i16).                  */
/* ------------------------------------------------------------------------ */
ORC_API float orc_quantize_act_u8(const float *x, int64_t k, uint8_t *out) {
    float mx = 0.f;
    for (int64_t i = 0; i < k; ++i) {
        float a = fabsf(x[i]);
        mx = a > mx ? a : mx;
    }
    if (mx < 1e-10f) mx = 1e-10f;
    float sx = mx / 127.0f, inv = 1.0f / sx;
    int64_t body = k / 16 * 16;
    for (int64_t i = 0; i < k; ++i) {
        float q;
        if (i < body) {
            q = nearbyintf(x[i] * inv);
        } else {
            q = roundf(x[i] / sx);
            q = q > 127.f ? 127.f : (q < -127.f ? -127.f : q);
        }
        out[i] = isnan(q) ? (uint8_t)128 : (uint8_t)((int32_t)q + 128);
    }
    return sx;
}

/* gemv_row_w4a8_group64_vnni_avx512 (gemv.rs:1422-1473; v2 block form       */
/* packed_v2.rs:204-241 and the 8-row form 288-323, same arithmetic per row): */
/* lane j of the 16 dpbusd lanes holds the exact integer sum over elements   */
/* 4j..4j+3 of (byte - 128) * (nib - 8); acc_j = fma((float)lane, s_x * s_w,  */
/* acc_j) per group; tree16 at the end.  blocked != 0: w holds v2 blocks.     */
/* With k % 64 != 0 (v1 only) the reference's last group reads past the row  */
/* and the activation bytes (undefined); here its missing elements count as  */
/* zero, the library's defined form.                                         */
HOT static void w4a8_rows(const uint8_t *xu, float sx, const uint8_t *w, const float *s,
                          int blocked, const float *bias, float *y, int64_t r0, int64_t r1,
                          int64_t k) {
    int64_t ng = (k + 63) / 64, bpr = (k + 1) / 2;
    for (int64_t r = r0; r < r1; ++r) {
        float acc[L16] = {0};
        for (int64_t g = 0; g < ng; ++g) {
            const uint8_t *nib = blocked ? w + (r * ng + g) * 34 : w + r * bpr + g * 32;
            float sw = blocked ? v2_scale(nib) : s[r * ng + g];
            float sc = sx * sw;
            for (int j = 0; j < L16; ++j) {
                int32_t t = 0;
                for (int e = 4 * j; e < 4 * j + 4; ++e) {
                    if (g * 64 + e >= k) break;
                    uint8_t b = nib[e / 2];
                    int32_t q = (int32_t)((e & 1) ? (b >> 4) : (b & 0x0F)) - 8;
                    t += ((int32_t)xu[g * 64 + e] - 128) * q;
                }
                acc[j] = fmaf((float)t, sc, acc[j]);
            }
        }
        y[r] = tree16(acc) + (bias ? bias[r] : 0.f);
    }
}

ORC_API void orc_gemv_w4a8_g64(const float *x, const uint8_t *w, const float *s, int blocked,
                               const float *bias, float *y, int64_t n, int64_t k) {
    uint8_t *xu = (uint8_t *)malloc((size_t)k);
    float sx = orc_quantize_act_u8(x, k, xu);
    int64_t ch = rayon_chunk(n);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t c = 0; c < (n + ch - 1) / ch; ++c)
        w4a8_rows(xu, sx, w, s, blocked, bias, y, c * ch, (c + 1) * ch < n ? (c + 1) * ch : n, k);
    free(xu);
}

/* ------------------------------------------------------------------------ */
/* a7/a8: SwiGLU.  Neuron pair swiglu.rs:205-255 (g32) / 85-163 (g64) is the   */
/* a4 row kernel applied to the gate and the up row with shared x;           */
/* h = silu(g + gb) * (u + ub), silu(g) = g / (1 + exp(-g))                  */
/* (fused_ops.rs:404-406).  Then down = gemv_w4a32_grouped(h)                 */
/* (fused_ops.rs:409-421).  The residual is the caller's (decoder.rs:1344).   */
/* ------------------------------------------------------------------------ */
HOT static void swiglu_w4_rows(const float *x, const uint8_t *gw, const float *gsc,
                               const float *gb, const uint8_t *uw, const float *usc,
                               const float *ub, float *h, int64_t j0, int64_t j1, int64_t k,
                               int64_t gs) {
    int64_t ng = (k + gs - 1) / gs, bpr = (k + 1) / 2;
    for (int64_t j = j0; j < j1; ++j) {
        float g = w4_row(x, gw + j * bpr, gsc + j * ng, k, gs) + (gb ? gb[j] : 0.f);
        float u = w4_row(x, uw + j * bpr, usc + j * ng, k, gs) + (ub ? ub[j] : 0.f);
        float silu = g / (1.0f + expf(-g));
        h[j] = silu * u;
    }
}

ORC_API void orc_swiglu_h_w4(const float *x, const uint8_t *gw, const float *gsc,
                             const float *gb, const uint8_t *uw, const float *usc,
                             const float *ub, float *h, int64_t inter, int64_t k, int64_t gs) {
    int64_t ch = rayon_chunk(inter);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t c = 0; c < (inter + ch - 1) / ch; ++c)
        swiglu_w4_rows(x, gw, gsc, gb, uw, usc, ub, h, c * ch,
                       (c + 1) * ch < inter ? (c + 1) * ch : inter, k, gs);
}

ORC_API void orc_swiglu_mlp_w4(const float *x, const uint8_t *gw, const float *gsc,
                               const float *gb, const uint8_t *uw, const float *usc,
                               const float *ub, const uint8_t *dw, const float *dsc,
                               const float *db, float *out, int64_t m, int64_t k,
                               int64_t inter, int64_t nout, int64_t gs) {
    float *h = (float *)malloc((size_t)inter * sizeof(float));
    for (int64_t t = 0; t < m; ++t) {
        orc_swiglu_h_w4(x + t * k, gw, gsc, gb, uw, usc, ub, h, inter, k, gs);
        orc_gemv_w4(h, dw, dsc, db, out + t * nout, nout, inter, gs);
    }
    free(h);
}

/* The W4A8 form at group 64 on an AVX-512 VNNI host (fused_ops.rs:215-232,   */
/* 409-421): x rounded to bytes per token; gate and up by                     */
/* swiglu_neuron_w4a8_group64_vnni_avx512 (swiglu.rs:8-81: per matrix the      */
/* lanes and per-group fma of gemv_row_w4a8_group64_vnni_avx512, w4a8_rows);   */
/* h = silu(g + gb) * (u + ub); the down projection is a group-64 GEMV, so W4A8 */
/* again on h.                                                                */
ORC_API void orc_swiglu_mlp_w4a8(const float *x, const uint8_t *gw, const float *gsc,
                                 const float *gb, const uint8_t *uw, const float *usc,
                                 const float *ub, const uint8_t *dw, const float *dsc,
                                 const float *db, float *out, int64_t m, int64_t k,
                                 int64_t inter, int64_t nout) {
    float *g = (float *)malloc((size_t)inter * sizeof(float));
    float *u = (float *)malloc((size_t)inter * sizeof(float));
    float *h = (float *)malloc((size_t)inter * sizeof(float));
    for (int64_t t = 0; t < m; ++t) {
        orc_gemv_w4a8_g64(x + t * k, gw, gsc, 0, NULL, g, inter, k);
        orc_gemv_w4a8_g64(x + t * k, uw, usc, 0, NULL, u, inter, k);
        for (int64_t j = 0; j < inter; ++j) {
            float gv = g[j] + (gb ? gb[j] : 0.f), uv = u[j] + (ub ? ub[j] : 0.f);
            h[j] = gv / (1.0f + expf(-gv)) * uv;
        }
        orc_gemv_w4a8_g64(h, dw, dsc, 0, db, out + t * nout, nout, inter);
    }
    free(g);
    free(u);
    free(h);
}

/* ------------------------------------------------------------------------ */
/* Per-channel INT4: w4a32_linear, gemv.rs:1066-1182 (the compile engine's    */
/* d_quant.rs:109-125 and python/torchburn/quantization.py:219-243):           */
/*   y[r] = dot_f32_u4(x, w[r], k) * s + b,  s = s[r] (or s[0] when 1 element) */
/* dot_f32_u4 AVX2 tier, gemv.rs:643-704: per 32-element chunk elements 0-7    */
/* and 16-23 feed accumulator 0, 8-15 and 24-31 accumulator 1 (8 lanes each,  */
/* fma); the two are added lane-wise, hsum256_ps_avx (gemv.rs:11-19: high +   */
/* low 128, then movehl, then lane 1 + lane 0), then the scalar tail adds     */
/* x * q element by element.                                                  */
/* ------------------------------------------------------------------------ */
static float hsum8(const float *v) {
    float s4[4];
    for (int i = 0; i < 4; ++i) s4[i] = v[i + 4] + v[i];
    float a = s4[0] + s4[2], b = s4[1] + s4[3];
    return a + b;
}

static inline float dot_f32_u4(const float *x, const uint8_t *w, int64_t len) {
    float s0[8] = {0}, s1[8] = {0};
    int64_t off = 0;
    for (; off + 32 <= len; off += 32) {
        float q[32];
        for (int j = 0; j < 16; ++j) {
            uint8_t b = w[off / 2 + j];
            q[2 * j] = (float)((int)(b & 15) - 8);
            q[2 * j + 1] = (float)((int)(b >> 4) - 8);
        }
        for (int l = 0; l < 8; ++l) s0[l] = fmaf(q[l], x[off + l], s0[l]);
        for (int l = 0; l < 8; ++l) s1[l] = fmaf(q[8 + l], x[off + 8 + l], s1[l]);
        for (int l = 0; l < 8; ++l) s0[l] = fmaf(q[16 + l], x[off + 16 + l], s0[l]);
        for (int l = 0; l < 8; ++l) s1[l] = fmaf(q[24 + l], x[off + 24 + l], s1[l]);
    }
    float sum[8];
    for (int l = 0; l < 8; ++l) sum[l] = s0[l] + s1[l];
    float t = hsum8(sum);
    for (; off < len; ++off) {
        uint8_t b = w[off / 2];
        int q = (off % 2 == 0) ? (int)(b & 15) - 8 : (int)(b >> 4) - 8;
        t += x[off] * (float)q;
    }
    return t;
}

ORC_API void orc_gemv_w4_rows(const float *x, const uint8_t *w, const float *s, int64_t s_len,
                              const float *bias, float *y, int64_t n, int64_t k) {
    int64_t bpr = (k + 1) / 2;
#pragma omp parallel for schedule(dynamic, 8)
    for (int64_t r = 0; r < n; ++r) {
        float sc = s_len > 1 ? s[r] : s[0];
        y[r] = dot_f32_u4(x, w + r * bpr, k) * sc + (bias ? bias[r] : 0.f);
    }
}

/* quantize_linear_weights_int4, fused_ops.rs:592-639: per row               */
/* s = amax / 7 (1 when amax <= 1e-8), inv = 1 / s,                           */
/* q = clamp(round_half_away(w * inv), -8, 7) + 8, two per byte (low nibble   */
/* first), an odd K's last byte padded with the nibble 8.                     */
ORC_API void orc_quantize_int4_rows(const float *w, uint8_t *packed, float *s, int64_t n,
                                    int64_t k) {
    int64_t kp = (k + 1) / 2;
    for (int64_t r = 0; r < n; ++r) {
        const float *row = w + r * k;
        float amax = 0.f;
        for (int64_t i = 0; i < k; ++i) {
            float a = fabsf(row[i]);
            if (a > amax) amax = a;
        }
        float sc = amax > 1e-8f ? amax / 7.0f : 1.0f;
        float inv = 1.0f / sc;
        s[r] = sc;
        for (int64_t b = 0; b < kp; ++b) {
            int q[2];
            for (int h = 0; h < 2; ++h) {
                int64_t e = 2 * b + h;
                if (e < k) {
                    /* f32::round, then clamp, which keeps a NaN, and `as i8`, */
                    /* which maps it to 0 (fused_ops.rs:620-629)               */
                    float v = roundf(row[e] * inv);
                    v = v < -8.f ? -8.f : (v > 7.f ? 7.f : v);
                    q[h] = isnan(v) ? 8 : (int)v + 8;
                } else {
                    q[h] = 8;
                }
            }
            packed[r * kp + b] = (uint8_t)((q[0] & 15) | ((q[1] & 15) << 4));
        }
    }
}

/* ------------------------------------------------------------------------ */
/* a18: INT8 W8A32.  dot_f32_i8_avx512 gemv.rs:280-324 and the 8-row kernel   */
/* gemv.rs:147-270 share one per-row structure: two 16-lane accumulators over */
/* 32-element chunks, summed, then 16-element chunks, lane reduce, scalar     */
/* tail.  Row result = dot * s + b (gemv.rs:777-785; s_len == 1 means one     */
/* per-tensor scale).                                                          */
/* ------------------------------------------------------------------------ */
static inline float dot_i8_row(const float *x, const int8_t *w, int64_t len) {
    float a0[L16] = {0}, a1[L16] = {0};
    int64_t off = 0;
    for (; off + 32 <= len; off += 32)
        for (int i = 0; i < L16; ++i) {
            a0[i] = fmaf((float)w[off + i], x[off + i], a0[i]);
            a1[i] = fmaf((float)w[off + 16 + i], x[off + 16 + i], a1[i]);
        }
    float sm[L16];
    for (int i = 0; i < L16; ++i) sm[i] = a0[i] + a1[i];
    for (; off + 16 <= len; off += 16)
        for (int i = 0; i < L16; ++i) sm[i] = fmaf((float)w[off + i], x[off + i], sm[i]);
    float t = tree16(sm);
    for (; off < len; ++off) t += x[off] * (float)w[off];
    return t;
}

HOT static void w8_rows(const float *x, const int8_t *w, const float *s, int64_t s_len,
                        const float *bias, float *y, int64_t r0, int64_t r1, int64_t k) {
    for (int64_t r = r0; r < r1; ++r) {
        float d = dot_i8_row(x, w + r * k, k);
        float sc = s_len > 1 ? s[r] : s[0];
        y[r] = d * sc + (bias ? bias[r] : 0.f);
    }
}

ORC_API void orc_gemv_w8(const float *x, const int8_t *w, const float *s, int64_t s_len,
                         const float *bias, float *y, int64_t n, int64_t k) {
    int64_t ch = rayon_chunk(n);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t c = 0; c < (n + ch - 1) / ch; ++c)
        w8_rows(x, w, s, s_len, bias, y, c * ch, (c + 1) * ch < n ? (c + 1) * ch : n, k);
}

/* Per-channel INT8 quantizer, fused_ops.rs:554-589: s = amax/127 (1 when    */
/* amax <= 1e-8), q = clamp(round_half_away(w * (1/s)), -127, 127).          */
ORC_API void orc_quantize_int8(const float *w, int8_t *q, float *s, int64_t n, int64_t k) {
    for (int64_t r = 0; r < n; ++r) {
        float amax = 0.f;
        for (int64_t i = 0; i < k; ++i) {
            float a = fabsf(w[r * k + i]);
            amax = a > amax ? a : amax;
        }
        float sc = amax > 1e-8f ? amax / 127.0f : 1.0f; /* fused_ops.rs:575 */
        float inv = 1.0f / sc;
        s[r] = sc;
        for (int64_t i = 0; i < k; ++i) {
            float v = roundf(w[r * k + i] * inv);
            v = v < -127.f ? -127.f : (v > 127.f ? 127.f : v);
            q[r * k + i] = (int8_t)v;
        }
    }
}

/* SwiGLU MLP with INT8 weights, fused_ops.rs:8-133: per neuron j            */
/*   g = dot(x, gate_j) * gs + gb,  u = dot(x, up_j) * us + ub                 */
/* (fused_ops.rs:101-105; a scale slice of one element is a per-tensor scalar, */
/* fused_ops.rs:80-97; absent biases are 0), h_j = silu(g) * u, then the INT8  */
/* down GEMV with its own scale length and bias (fused_ops.rs:117-128).        */
HOT static void swiglu_w8_rows(const float *x, const int8_t *gw, const float *gsc,
                               int64_t gs_len, const float *gb, const int8_t *uw,
                               const float *usc, int64_t us_len, const float *ub, float *h,
                               int64_t j0, int64_t j1, int64_t k) {
    for (int64_t j = j0; j < j1; ++j) {
        float gsj = gs_len > 1 ? gsc[j] : gsc[0];
        float usj = us_len > 1 ? usc[j] : usc[0];
        float g = dot_i8_row(x, gw + j * k, k) * gsj + (gb ? gb[j] : 0.f);
        float u = dot_i8_row(x, uw + j * k, k) * usj + (ub ? ub[j] : 0.f);
        float silu = g / (1.0f + expf(-g));
        h[j] = silu * u;
    }
}

ORC_API void orc_swiglu_h_w8(const float *x, const int8_t *gw, const float *gsc, int64_t gs_len,
                             const float *gb, const int8_t *uw, const float *usc,
                             int64_t us_len, const float *ub, float *h, int64_t inter,
                             int64_t k) {
    int64_t ch = rayon_chunk(inter);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t c = 0; c < (inter + ch - 1) / ch; ++c)
        swiglu_w8_rows(x, gw, gsc, gs_len, gb, uw, usc, us_len, ub, h, c * ch,
                       (c + 1) * ch < inter ? (c + 1) * ch : inter, k);
}

/* fused_swiglu_mlp_w8a32 over m tokens (fused_ops.rs:52-131: one token at a  */
/* time, h then gemv_w8a32 of the down projection).                           */
ORC_API void orc_swiglu_mlp_w8(const float *x, const int8_t *gw, const float *gsc,
                               int64_t gs_len, const float *gb, const int8_t *uw,
                               const float *usc, int64_t us_len, const float *ub,
                               const int8_t *dw, const float *dsc, int64_t ds_len,
                               const float *db, float *out, int64_t m, int64_t k, int64_t inter,
                               int64_t nout) {
    float *h = (float *)malloc((size_t)(inter > 0 ? inter : 1) * sizeof(float));
    for (int64_t t = 0; t < m; ++t) {
        orc_swiglu_h_w8(x + t * k, gw, gsc, gs_len, gb, uw, usc, us_len, ub, h, inter, k);
        orc_gemv_w8(h, dw, dsc, ds_len, db, out + t * nout, nout, inter);
    }
    free(h);
}

/* ------------------------------------------------------------------------ */
/* a9: fast_rms_norm AVX-512 tier, fused_ops.rs:1066-1089.                    */
/* ------------------------------------------------------------------------ */
ORC_API void orc_rms_norm(const float *x, const float *w, float *out, int64_t n, float eps) {
    float acc[L16] = {0};
    int64_t nc = n / 16;
    for (int64_t c = 0; c < nc; ++c)
        for (int i = 0; i < L16; ++i) acc[i] = fmaf(x[c * 16 + i], x[c * 16 + i], acc[i]);
    float tot = tree16(acc);
    for (int64_t i = nc * 16; i < n; ++i) tot += x[i] * x[i];
    float rms = sqrtf(tot / (float)n + eps);
    float inv = 1.0f / rms;
    for (int64_t i = 0; i < nc * 16; ++i) out[i] = (x[i] * inv) * w[i];
    for (int64_t i = nc * 16; i < n; ++i) out[i] = (x[i] / rms) * w[i];
}

/* RMSNorm of the reference's per-layer Python path, python/torchburn/llm/    */
/* model.py:91-98 (F.rms_norm): y = (x * rsqrt(mean(x^2) + eps)) * w in f32.  */
/* The sum of squares is taken in 16 lanes and a tree, as a vectorised CPU    */
/* reduction does; torch's exact lane order is not pinned at the bit level.   */
ORC_API void orc_rms_norm_torch(const float *x, const float *w, float *out, int64_t n,
                                float eps) {
    float acc[L16] = {0};
    int64_t nc = n / 16;
    for (int64_t c = 0; c < nc; ++c)
        for (int i = 0; i < L16; ++i) acc[i] = fmaf(x[c * 16 + i], x[c * 16 + i], acc[i]);
    float tot = tree16(acc);
    for (int64_t i = nc * 16; i < n; ++i) tot += x[i] * x[i];
    float r = 1.0f / sqrtf(tot / (float)n + eps);
    for (int64_t i = 0; i < n; ++i) out[i] = (x[i] * r) * w[i];
}

/* dot_f32_f32 AVX-512 tier, fused_ops.rs:646-664 (len >= 16), else scalar.  */
static inline float dot_f32(const float *a, const float *b, int64_t len) {
    if (len >= 16) {
        float acc[L16] = {0};
        int64_t i = 0;
        for (; i + 16 <= len; i += 16)
            for (int l = 0; l < L16; ++l) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
        float s = tree16(acc);
        for (; i < len; ++i) s += a[i] * b[i];
        return s;
    }
    float s = 0.f;
    for (int64_t i = 0; i < len; ++i) s += a[i] * b[i];
    return s;
}

/* FP32 linear (the fp32 lm_head of the per-layer Python path,               */
/* python/torchburn/llm/model.py:499-500): y[r] = dot(W[r], x).  torch's CPU  */
/* sgemv order is not pinned; the row dot above stands for it.               */
HOT static void f32_rows(const float *x, const float *w, float *y, int64_t r0, int64_t r1,
                         int64_t k) {
    for (int64_t r = r0; r < r1; ++r) y[r] = dot_f32(w + r * k, x, k);
}

ORC_API void orc_gemv_f32(const float *x, const float *w, float *y, int64_t n, int64_t k) {
    int64_t ch = rayon_chunk(n);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t c = 0; c < (n + ch - 1) / ch; ++c)
        f32_rows(x, w, y, c * ch, (c + 1) * ch < n ? (c + 1) * ch : n, k);
}

/* ------------------------------------------------------------------------ */
/* a10: RoPE.  Tables decoder.rs:334-350 (f64 math, cast to f32, both halves  */
/* duplicated); rotate-half apply decoder.rs:28-68 (mul and sub separately).  */
/* ------------------------------------------------------------------------ */
ORC_API void orc_rope_tables(float *cos_t, float *sin_t, int64_t max_seq, int64_t hd,
                             double theta) {
    int64_t half = hd / 2;
    for (int64_t p = 0; p < max_seq; ++p)
        for (int64_t i = 0; i < half; ++i) {
            double freq = 1.0 / pow(theta, (2.0 * (double)i) / (double)hd);
            double val = (double)p * freq;
            float c = (float)cos(val), s = (float)sin(val);
            cos_t[p * hd + i] = cos_t[p * hd + i + half] = c;
            sin_t[p * hd + i] = sin_t[p * hd + i + half] = s;
        }
}

ORC_API void orc_rope_apply(float *head, const float *c, const float *s, int64_t half) {
    for (int64_t i = 0; i < half; ++i) {
        float x1 = head[i], x2 = head[i + half];
        head[i] = x1 * c[i] - x2 * s[i];
        head[i + half] = x2 * c[i + half] + x1 * s[i + half];
    }
}

/* ------------------------------------------------------------------------ */
/* a12: GQA decode attention for one query head, decoder.rs:1148-1213.        */
/* kv_base points at [seq, hd] rows of this head's KV.                       */
/* ------------------------------------------------------------------------ */
/* max_pos: the native step's cap, 32768 (decoder.rs:1179-1184); the oracle   */
/* decoder takes another value only through orc_decoder_set_attention_cap.   */
static void attend_head(const float *q, const float *kb, const float *vb, float *out,
                        float *scores, int64_t seq_len, int64_t hd, int64_t max_pos) {
    for (int64_t d = 0; d < hd; ++d) out[d] = 0.f;
    if (seq_len == 1) {
        memcpy(out, vb, (size_t)hd * sizeof(float));
        return;
    }
    int64_t cap = seq_len < max_pos ? seq_len : max_pos;
    float scale = 1.0f / sqrtf((float)hd);
    float mx = -INFINITY;
    for (int64_t t = 0; t < cap; ++t) {
        float sc = dot_f32(q, kb + t * hd, hd) * scale;
        scores[t] = sc;
        if (sc > mx) mx = sc;
    }
    float sum = 0.f;
    for (int64_t t = 0; t < cap; ++t) {
        float e = expf(scores[t] - mx);
        scores[t] = e;
        sum += e;
    }
    float inv = 1.0f / (sum > 1e-30f ? sum : 1e-30f);
    for (int64_t t = 0; t < cap; ++t) {
        float wt = scores[t] * inv;
        const float *v = vb + t * hd;
        /* fast_vector_fma AVX-512 tier, fused_ops.rs:1189-1202 */
        int64_t nc = hd / 16;
        for (int64_t i = 0; i < nc * 16; ++i) out[i] = fmaf(wt, v[i], out[i]);
        for (int64_t i = nc * 16; i < hd; ++i) out[i] += wt * v[i];
    }
}

/* The attention of the per-layer steps, fused_ops.rs:997-1040 (INT4) and     */
/* 823-858 (INT8): every position 0..seq_len-1 (no single-position shortcut,  */
/* no 32768 cap), inv = 1 / sum with no clamp, out += w * v rounded twice.    */
static void attend_head_layer(const float *q, const float *kb, const float *vb, float *out,
                              float *scores, int64_t seq_len, int64_t hd) {
    for (int64_t d = 0; d < hd; ++d) out[d] = 0.f;
    float scale = 1.0f / sqrtf((float)hd);
    float mx = -INFINITY;
    for (int64_t t = 0; t < seq_len; ++t) {
        float sc = dot_f32(q, kb + t * hd, hd) * scale;
        scores[t] = sc;
        if (sc > mx) mx = sc;
    }
    float sum = 0.f;
    for (int64_t t = 0; t < seq_len; ++t) {
        float e = expf(scores[t] - mx);
        scores[t] = e;
        sum += e;
    }
    float inv = 1.0f / sum;
    for (int64_t t = 0; t < seq_len; ++t) {
        float wt = scores[t] * inv;
        const float *v = vb + t * hd;
        for (int64_t d = 0; d < hd; ++d) out[d] += wt * v[d];
    }
}

/* q: [hq, hd]; k_cache/v_cache: [hkv, max_seq, hd]; out: [hq, hd]. */
static void attention_any(const float *q, const float *k_cache, const float *v_cache,
                          float *out, int64_t hq, int64_t hkv, int64_t hd, int64_t max_seq,
                          int64_t seq_len, int layer_path, int64_t max_pos) {
    int64_t per = hq / (hkv > 0 ? hkv : 1);
    if (per < 1) per = 1;
#pragma omp parallel
    {
        float *scores = (float *)malloc((size_t)(seq_len > 0 ? seq_len : 1) * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t h = 0; h < hq; ++h) {
            int64_t kvh = h / per;
            if (layer_path)
                attend_head_layer(q + h * hd, k_cache + kvh * max_seq * hd,
                                  v_cache + kvh * max_seq * hd, out + h * hd, scores, seq_len, hd);
            else
                attend_head(q + h * hd, k_cache + kvh * max_seq * hd,
                            v_cache + kvh * max_seq * hd, out + h * hd, scores, seq_len, hd,
                            max_pos);
        }
        free(scores);
    }
}

ORC_API void orc_attention(const float *q, const float *k_cache, const float *v_cache,
                           float *out, int64_t hq, int64_t hkv, int64_t hd, int64_t max_seq,
                           int64_t seq_len) {
    attention_any(q, k_cache, v_cache, out, hq, hkv, hd, max_seq, seq_len, 0, 32768);
}

/* The per-layer steps' attention (attend_head_layer) for q [hq, hd]. */
ORC_API void orc_attention_layer(const float *q, const float *k_cache, const float *v_cache,
                                 float *out, int64_t hq, int64_t hkv, int64_t hd,
                                 int64_t max_seq, int64_t seq_len) {
    attention_any(q, k_cache, v_cache, out, hq, hkv, hd, max_seq, seq_len, 1, 32768);
}

/* a17: greedy argmax, decoder.rs:914-925 (strict >, lowest index wins).      */
ORC_API int64_t orc_argmax(const float *v, int64_t n) {
    if (n <= 0) return 0;
    int64_t bi = 0;
    float bv = v[0];
    for (int64_t i = 1; i < n; ++i)
        if (v[i] > bv) {
            bv = v[i];
            bi = i;
        }
    return bi;
}

/* ------------------------------------------------------------------------ */
/* f4: sampling.  apply_repetition_penalty, decoder.rs:878-899: each distinct */
/* in-vocabulary recent token's logit / penalty when > 0, else * penalty.     */
/* ------------------------------------------------------------------------ */
ORC_API void orc_repetition_penalty(float *logits, int64_t V, const int64_t *recent, int64_t n,
                                    float penalty) {
    if (!(penalty > 1.0f) || n <= 0) return;
    for (int64_t i = 0; i < n; ++i) {
        int64_t t = recent[i], dup = 0;
        if (t < 0 || t >= V) continue;
        for (int64_t j = 0; j < i && !dup; ++j) dup = recent[j] == t;
        if (dup) continue;
        float l = logits[t];
        logits[t] = l > 0.f ? l / penalty : l * penalty;
    }
}

/* sample_logits, decoder.rs:908-1020, with the uniform u supplied:          */
/*  greedy (temperature not finite or <= 0, or top_k == 1): orc_argmax, the  */
/*  reference's scan from logits[0] with strict > (a NaN at index 0 wins, a  */
/*  NaN elsewhere is never chosen);                                          */
/*  else k = clamp(top_k, 1, V) candidates, non-finite logits as -inf, taken */
/*  by (value descending, index ascending) and visited in that order;         */
/*  p_i = exp((v_i - v_0) * (1/T)); nucleus: keep while the normalised mass  */
/*  before the item is <= top_p (0 < top_p < 1); r = u * kept mass; first    */
/*  item whose running mass >= r.  *kept_out = candidates after top-k.       */
typedef struct { float v; int64_t i; } orc_item;
static int item_cmp(const void *a, const void *b) {
    const orc_item *x = (const orc_item *)a, *y = (const orc_item *)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return x->i < y->i ? -1 : (x->i > y->i);
}

ORC_API int64_t orc_sample_logits(const float *logits, int64_t V, float temperature,
                                  int64_t top_k, float top_p, float u, int64_t *kept_out) {
    if (V <= 0) return 0;
    if (!isfinite(temperature) || temperature <= 0.f || top_k == 1) {
        if (kept_out) *kept_out = 1;
        return orc_argmax(logits, V); /* decoder.rs:914-925: a NaN at index 0 wins */
    }
    int64_t k = top_k < 1 ? 1 : (top_k > V ? V : top_k);
    orc_item *it = (orc_item *)malloc((size_t)V * sizeof(orc_item));
    for (int64_t i = 0; i < V; ++i) {
        it[i].v = isfinite(logits[i]) ? logits[i] : -INFINITY;
        it[i].i = i;
    }
    qsort(it, (size_t)V, sizeof(orc_item), item_cmp);
    float *p = (float *)malloc((size_t)k * sizeof(float));
    float mx = it[0].v, inv_t = 1.0f / temperature, pre = 0.f;
    for (int64_t i = 0; i < k; ++i) {
        p[i] = expf((it[i].v - mx) * inv_t);
        pre += p[i];
    }
    int64_t kept = k;
    if (top_p > 0.f && top_p < 1.f && k > 1 && pre > 0.f) {
        float inv = 1.0f / pre, cum = 0.f;
        for (int64_t i = 0; i < k; ++i) {
            if (cum > top_p) {
                kept = i;
                break;
            }
            cum += p[i] * inv;
        }
    }
    float ks = 0.f;
    for (int64_t i = 0; i < kept; ++i) ks += p[i];
    float r = u * ks, acc = 0.f;
    int64_t tok = it[0].i;
    for (int64_t i = 0; i < kept; ++i) {
        acc += p[i];
        if (acc >= r) {
            tok = it[i].i;
            break;
        }
    }
    if (kept_out) *kept_out = k;
    free(p);
    free(it);
    return tok;
}

/* speculative_accept's acceptance, decoder.rs:608-726, over target rows     */
/* [K, V] and draft_probs [K, V] with the uniforms u[] consumed in order:     */
/* per position the temperature softmax (non-finite -> -inf, sum clamped at  */
/* 1e-30), accept while u <= min(p_t[d] / (p_d[d] + 1e-12), 1); on reject    */
/* the bonus is drawn from max(0, p_t - p_d) in index order (argmax of p_t   */
/* when its mass is <= 1e-12); all accepted: the bonus from the last row's   */
/* distribution by probability (ties: lower index), nucleus-cut at top_p.    */
static void orc_softmax_t(const float *lg, int64_t V, float temp, float *p) {
    float t = (isfinite(temp) && temp > 0.f) ? temp : 1.0f, m = -INFINITY, s = 0.f;
    for (int64_t j = 0; j < V; ++j) {
        float v = isfinite(lg[j]) ? lg[j] : -INFINITY;
        m = v > m ? v : m;
    }
    for (int64_t j = 0; j < V; ++j) {
        p[j] = expf(((isfinite(lg[j]) ? lg[j] : -INFINITY) - m) / t);
        s += p[j];
    }
    float inv = 1.0f / (s > 1e-30f ? s : 1e-30f);
    for (int64_t j = 0; j < V; ++j) p[j] *= inv;
}

static const float *g_sort_p;
static int prob_desc(const void *a, const void *b) {
    int64_t x = *(const int64_t *)a, y = *(const int64_t *)b;
    if (g_sort_p[x] > g_sort_p[y]) return -1;
    if (g_sort_p[x] < g_sort_p[y]) return 1;
    return x < y ? -1 : (x > y);
}

ORC_API void orc_speculative_accept(const float *rows, const int64_t *draft, const float *dp,
                                    int64_t K, int64_t V, float temperature, float top_p,
                                    const double *u, int64_t n_u, int64_t *accepted,
                                    int64_t *bonus) {
    int64_t ui = 0;
#define NEXT_U() (ui < n_u ? u[ui++] : 0.0)
    *accepted = 0;
    *bonus = V - 1;
    if (K == 0) return;
    float *tp = (float *)malloc((size_t)V * sizeof(float));
    for (int64_t i = 0; i < K; ++i) {
        orc_softmax_t(rows + i * V, V, temperature, tp);
        int64_t d = draft[i] < 0 ? 0 : (draft[i] > V - 1 ? V - 1 : draft[i]);
        float pt = tp[d], pd = dp[i * V + d] > 0.f ? dp[i * V + d] : 0.f;
        float acc = pt / (pd + 1e-12f);
        if (acc > 1.f) acc = 1.f;
        if (NEXT_U() <= (double)acc) {
            *accepted += 1;
            continue;
        }
        float sc = 0.f;
        for (int64_t j = 0; j < V; ++j) {
            float c = tp[j] - dp[i * V + j];
            sc += c > 0.f ? c : 0.f;
        }
        if (sc > 1e-12f) {
            float r = (float)NEXT_U() * sc, a = 0.f;
            *bonus = V - 1;
            for (int64_t j = 0; j < V; ++j) {
                float c = tp[j] - dp[i * V + j];
                a += c > 0.f ? c : 0.f;
                if (a >= r) {
                    *bonus = j;
                    break;
                }
            }
        } else {
            int64_t bj = 0;
            for (int64_t j = 1; j < V; ++j)
                if (tp[j] > tp[bj]) bj = j;
            *bonus = bj;
        }
        free(tp);
        return;
    }
    orc_softmax_t(rows + (K - 1) * V, V, temperature, tp);
    int64_t *idx = (int64_t *)malloc((size_t)V * sizeof(int64_t));
    for (int64_t j = 0; j < V; ++j) idx[j] = j;
    g_sort_p = tp;
    qsort(idx, (size_t)V, sizeof(int64_t), prob_desc);
    int64_t kept = V;
    if (top_p > 0.f && top_p < 1.f) {
        float cum = 0.f;
        for (int64_t i = 0; i < V; ++i) {
            if (cum > top_p) {
                kept = i;
                break;
            }
            cum += tp[idx[i]];
        }
        if (kept < 1) kept = 1;
    }
    float mass = 0.f;
    for (int64_t i = 0; i < kept; ++i) mass += tp[idx[i]];
    float r = (float)NEXT_U() * (mass > 1e-30f ? mass : 1e-30f), a = 0.f;
    *bonus = idx[kept - 1];
    for (int64_t i = 0; i < kept; ++i) {
        a += tp[idx[i]];
        if (a >= r) {
            *bonus = idx[i];
            break;
        }
    }
#undef NEXT_U
    free(idx);
    free(tp);
}

/* ------------------------------------------------------------------------ */
/* a16: RustQwenDecoder::step_internal, decoder.rs:1051-1374.                 */
/* The oracle borrows every weight pointer (the caller keeps them alive) and */
/* owns its KV cache [L][hkv, max_seq, hd], RoPE tables and scratch, as the  */
/* reference does (decoder.rs:334-359).                                      */
/* wkind: 4 = INT4 grouped (the native decoder), 8 = INT8 per-channel        */
/*   projections with the same step structure (the reference has no native   */
/*   INT8 decoder; engine.py:133-151 routes INT8 through the per-layer path  */
/*   whose GEMVs are the a18 kernels).                                        */
/* lmkind: 4 = INT4 grouped, 8 = INT8 per-channel, 32 = fp32.                 */
/* ------------------------------------------------------------------------ */
typedef struct {
    const float *in_norm, *post_norm;
    const void *qkv_w, *o_w, *gate_w, *up_w, *down_w;
    const float *qkv_s, *o_s, *gate_s, *up_s, *down_s;
    const float *qkv_b; /* may be NULL */
    uint8_t *qkv_w2, *o_w2, *down_w2; /* owned v2 blocks (use_v2) */
} orc_layer;

typedef struct {
    int64_t L, H, I, hq, hkv, hd, V, gs, max_seq;
    int wkind, lmkind;
    int use_v2;     /* decoder.rs:361-390 */
    int layer_path; /* numerics of the per-layer Python path (orc_decoder_set_layer_path) */
    int64_t attn_cap; /* native step: positions scored, 32768 (orc_decoder_set_attention_cap) */
    int a8;         /* W4A8 on a VNNI host at group 64 (orc_decoder_set_a8)             */
    uint8_t *lm_w2;
    float eps;
    const float *embed, *final_norm;
    const void *lm_w;
    const float *lm_s;
    orc_layer *layers;
    float *kc, *vc, *cos_t, *sin_t;
    float *x, *xn, *qkv, *att, *o, *h, *dn, *logits;
    float *g; /* [I] gate row of the W4A8 SwiGLU */
    int64_t kv_used;
} orc_decoder;

ORC_API orc_decoder *orc_decoder_create(int64_t L, int64_t H, int64_t I, int64_t hq,
                                        int64_t hkv, int64_t hd, int64_t V, int64_t gs,
                                        int64_t max_seq, double theta, float eps, int wkind,
                                        int lmkind, const float *embed,
                                        const float *final_norm, const void *lm_w,
                                        const float *lm_s) {
    orc_decoder *d = (orc_decoder *)calloc(1, sizeof(orc_decoder));
    d->L = L; d->H = H; d->I = I; d->hq = hq; d->hkv = hkv; d->hd = hd; d->V = V;
    d->gs = gs; d->max_seq = max_seq; d->eps = eps; d->wkind = wkind; d->lmkind = lmkind;
    d->attn_cap = 32768;
    d->embed = embed; d->final_norm = final_norm; d->lm_w = lm_w; d->lm_s = lm_s;
    d->layers = (orc_layer *)calloc((size_t)L, sizeof(orc_layer));
    size_t kvn = (size_t)L * (size_t)hkv * (size_t)max_seq * (size_t)hd;
    d->kc = (float *)calloc(kvn, sizeof(float));
    d->vc = (float *)calloc(kvn, sizeof(float));
    d->cos_t = (float *)malloc((size_t)(max_seq * hd) * sizeof(float));
    d->sin_t = (float *)malloc((size_t)(max_seq * hd) * sizeof(float));
    orc_rope_tables(d->cos_t, d->sin_t, max_seq, hd, theta);
    int64_t tq = (hq + 2 * hkv) * hd;
    /* decoder.rs:361-390: group 64 with hidden, QKV rows, num_heads * head_dim,
     * intermediate and vocab all multiples of 64 -> QKV, O, down and lm_head run
     * the v2 GEMV on blocks repacked at load (f16 scales); gate / up stay v1.
     * (The reference passes the output width as the pack's row length for QKV and
     * lm_head; the pack copies 32-byte chunks and scales in one running order, so
     * the bytes are the same as with the true row length.) */
    d->use_v2 = wkind == 4 && gs == 64 && H % 64 == 0 && tq % 64 == 0 && (hq * hd) % 64 == 0 &&
                I % 64 == 0 && V % 64 == 0;
    if (d->use_v2 && lmkind == 4) {
        d->lm_w2 = (uint8_t *)malloc((size_t)V * (size_t)(H / 64) * 34);
        orc_pack_v1_to_v2((const uint8_t *)lm_w, lm_s, d->lm_w2, V, H);
    }
    d->x = (float *)calloc((size_t)H, 4);
    d->xn = (float *)calloc((size_t)H, 4);
    d->qkv = (float *)calloc((size_t)tq, 4);
    d->att = (float *)calloc((size_t)(hq * hd), 4);
    d->o = (float *)calloc((size_t)H, 4);
    d->g = (float *)calloc((size_t)I, 4);
    d->h = (float *)calloc((size_t)I, 4);
    d->dn = (float *)calloc((size_t)H, 4);
    d->logits = (float *)calloc((size_t)V, 4);
    return d;
}

ORC_API void orc_decoder_set_layer(orc_decoder *d, int64_t l, const float *in_norm,
                                   const void *qkv_w, const float *qkv_s, const void *o_w,
                                   const float *o_s, const float *post_norm,
                                   const void *gate_w, const float *gate_s, const void *up_w,
                                   const float *up_s, const void *down_w, const float *down_s,
                                   const float *qkv_b) {
    orc_layer *y = &d->layers[l];
    y->in_norm = in_norm; y->qkv_w = qkv_w; y->qkv_s = qkv_s; y->o_w = o_w; y->o_s = o_s;
    y->post_norm = post_norm; y->gate_w = gate_w; y->gate_s = gate_s; y->up_w = up_w;
    y->up_s = up_s; y->down_w = down_w; y->down_s = down_s; y->qkv_b = qkv_b;
    if (d->use_v2) {
        int64_t H = d->H, I = d->I, qd = d->hq * d->hd, tq = qd + 2 * d->hkv * d->hd;
        free(y->qkv_w2); free(y->o_w2); free(y->down_w2);
        y->qkv_w2 = (uint8_t *)malloc((size_t)tq * (size_t)(H / 64) * 34);
        y->o_w2 = (uint8_t *)malloc((size_t)H * (size_t)(qd / 64) * 34);
        y->down_w2 = (uint8_t *)malloc((size_t)H * (size_t)(I / 64) * 34);
        orc_pack_v1_to_v2((const uint8_t *)qkv_w, qkv_s, y->qkv_w2, tq, H);
        orc_pack_v1_to_v2((const uint8_t *)o_w, o_s, y->o_w2, H, qd);
        orc_pack_v1_to_v2((const uint8_t *)down_w, down_s, y->down_w2, H, I);
    }
}

ORC_API void orc_decoder_destroy(orc_decoder *d) {
    if (!d) return;
    for (int64_t l = 0; l < d->L; ++l) {
        free(d->layers[l].qkv_w2); free(d->layers[l].o_w2); free(d->layers[l].down_w2);
    }
    free(d->lm_w2);
    free(d->layers); free(d->kc); free(d->vc); free(d->cos_t); free(d->sin_t);
    free(d->x); free(d->xn); free(d->qkv); free(d->att); free(d->o); free(d->h); free(d->g);
    free(d->dn); free(d->logits); free(d);
}

ORC_API float *orc_decoder_logits(orc_decoder *d) { return d->logits; }
ORC_API float *orc_decoder_k_cache(orc_decoder *d, int64_t l) {
    return d->kc + l * d->hkv * d->max_seq * d->hd;
}
ORC_API float *orc_decoder_v_cache(orc_decoder *d, int64_t l) {
    return d->vc + l * d->hkv * d->max_seq * d->hd;
}
ORC_API int64_t orc_decoder_kv_len(orc_decoder *d) { return d->kv_used; }
ORC_API void orc_decoder_set_kv_len(orc_decoder *d, int64_t n) {
    if (n > d->kv_used) d->kv_used = n;
}

/* Caller-built RoPE tables [max_seq, hd] replace the f64 ones of           */
/* decoder.rs:334-350: the per-layer Python path takes cos / sin from         */
/* RotaryEmbedding (python/torchburn/llm/model.py:108-122), whose angle       */
/* pos * inv_freq is an f32 product.                                          */
ORC_API void orc_decoder_set_rope_tables(orc_decoder *d, const float *cos_t,
                                         const float *sin_t) {
    memcpy(d->cos_t, cos_t, (size_t)(d->max_seq * d->hd) * sizeof(float));
    memcpy(d->sin_t, sin_t, (size_t)(d->max_seq * d->hd) * sizeof(float));
}

/* 1: the step composes the per-layer Python path that the reference runs    */
/* when its native decoder does not apply (INT8 weights or an fp32 lm_head,  */
/* python/torchburn/llm/engine.py:133-151): F.rms_norm (model.py:91-98,      */
/* orc_rms_norm_torch) and the per-layer steps' attention (fused_ops.rs:      */
/* 823-858, 997-1040); the residual adds, projections and MLP are the same   */
/* kernels as the native step.  0 (default): RustQwenDecoder::step_internal. */
ORC_API void orc_decoder_set_layer_path(orc_decoder *d, int on) { d->layer_path = on; }

/* 1: the step of an AVX-512 VNNI host at group 64: every INT4 projection      */
/* takes its input's bytes, W4A8 (decoder.rs:1262-1282 for the SwiGLU pair;   */
/* projection_gemv, decoder.rs:1029-1049, into packed_v2.rs:366-370 for the   */
/* v2 projections or gemv.rs:1559-1563 for v1).  Used when wkind == 4 and      */
/* gs == 64; the lm_head too when lmkind == 4.                                */
ORC_API void orc_decoder_set_a8(orc_decoder *d, int on) { d->a8 = on; }

/* The native step scores positions 0 .. min(offset + 1, cap) - 1; the        */
/* reference's cap is the constant 32768 (decoder.rs:1179-1184), the default. */
/* Another value lets a test show the cap's effect on a short cache.          */
ORC_API void orc_decoder_set_attention_cap(orc_decoder *d, int64_t cap) {
    d->attn_cap = cap > 0 ? cap : 32768;
}

/* projection_gemv, decoder.rs:1029-1049 (v1 path). */
static void proj(const orc_decoder *d, int kind, const float *x, const void *w, const float *s,
                 const float *b, float *y, int64_t n, int64_t k) {
    if (kind == 4)
        orc_gemv_w4(x, (const uint8_t *)w, s, b, y, n, k, d->gs);
    else if (kind == 8)
        orc_gemv_w8(x, (const int8_t *)w, s, n, b, y, n, k);
    else {
        orc_gemv_f32(x, (const float *)w, y, n, k);
        if (b)
            for (int64_t i = 0; i < n; ++i) y[i] += b[i];
    }
}

/* An INT4 projection of the step: v2 blocks (use_v2) or v1, W4A8 under a8.  */
static void proj4(const orc_decoder *d, const float *x, const uint8_t *w1, const float *s1,
                  const uint8_t *w2, const float *b, float *y, int64_t n, int64_t k) {
    int a8 = d->a8 && d->gs == 64;
    if (w2 && a8)
        orc_gemv_w4a8_g64(x, w2, NULL, 1, b, y, n, k);
    else if (w2)
        orc_gemv_w4_v2(x, w2, b, y, n, k);
    else if (a8)
        orc_gemv_w4a8_g64(x, w1, s1, 0, b, y, n, k);
    else
        orc_gemv_w4(x, w1, s1, b, y, n, k, d->gs);
}

ORC_API void orc_decoder_step(orc_decoder *d, int64_t token, int64_t offset) {
    int64_t H = d->H, hd = d->hd, hq = d->hq, hkv = d->hkv;
    int64_t qd = hq * hd, kvd = hkv * hd, tq = qd + 2 * kvd, half = hd / 2;
    /* decoder.rs:1066-1089: out-of-range token or offset -> zeroed step. */
    if (token < 0 || token >= d->V || offset < 0 || offset >= d->max_seq) {
        memset(d->x, 0, (size_t)H * 4);
        memset(d->logits, 0, (size_t)d->V * 4);
        return;
    }
    memcpy(d->x, d->embed + token * H, (size_t)H * 4);
    const float *cp = d->cos_t + offset * hd, *sp = d->sin_t + offset * hd;
    if (offset + 1 > d->kv_used) d->kv_used = offset + 1;
    for (int64_t l = 0; l < d->L; ++l) {
        const orc_layer *y = &d->layers[l];
        if (d->layer_path)
            orc_rms_norm_torch(d->x, y->in_norm, d->xn, H, d->eps);
        else
            orc_rms_norm(d->x, y->in_norm, d->xn, H, d->eps);
        if (d->wkind == 4)
            proj4(d, d->xn, (const uint8_t *)y->qkv_w, y->qkv_s, d->use_v2 ? y->qkv_w2 : NULL,
                  y->qkv_b, d->qkv, tq, H);
        else
            proj(d, d->wkind, d->xn, y->qkv_w, y->qkv_s, y->qkv_b, d->qkv, tq, H);
        float *q = d->qkv, *k = d->qkv + qd, *v = d->qkv + qd + kvd;
        for (int64_t h = 0; h < hq; ++h) orc_rope_apply(q + h * hd, cp, sp, half);
        for (int64_t h = 0; h < hkv; ++h) orc_rope_apply(k + h * hd, cp, sp, half);
        float *kc = orc_decoder_k_cache(d, l), *vc = orc_decoder_v_cache(d, l);
        for (int64_t h = 0; h < hkv; ++h) {
            memcpy(kc + (h * d->max_seq + offset) * hd, k + h * hd, (size_t)hd * 4);
            memcpy(vc + (h * d->max_seq + offset) * hd, v + h * hd, (size_t)hd * 4);
        }
        attention_any(q, kc, vc, d->att, hq, hkv, hd, d->max_seq, offset + 1, d->layer_path,
                      d->attn_cap);
        if (d->wkind == 4)
            proj4(d, d->att, (const uint8_t *)y->o_w, y->o_s, d->use_v2 ? y->o_w2 : NULL, NULL,
                  d->o, H, qd);
        else
            proj(d, d->wkind, d->att, y->o_w, y->o_s, NULL, d->o, H, qd);
        for (int64_t i = 0; i < H; ++i) d->x[i] += d->o[i];
        if (d->layer_path)
            orc_rms_norm_torch(d->x, y->post_norm, d->xn, H, d->eps);
        else
            orc_rms_norm(d->x, y->post_norm, d->xn, H, d->eps);
        if (d->wkind == 4 && d->a8 && d->gs == 64) {
            /* swiglu_neuron_w4a8_group64_vnni_avx512 (swiglu.rs:8-81): the W4A8  */
            /* row of each matrix on the same bytes, then silu(g) * u             */
            orc_gemv_w4a8_g64(d->xn, (const uint8_t *)y->gate_w, y->gate_s, 0, NULL, d->g, d->I,
                              H);
            orc_gemv_w4a8_g64(d->xn, (const uint8_t *)y->up_w, y->up_s, 0, NULL, d->h, d->I, H);
            for (int64_t j = 0; j < d->I; ++j) d->h[j] = d->g[j] / (1.0f + expf(-d->g[j])) * d->h[j];
        } else if (d->wkind == 4)
            orc_swiglu_h_w4(d->xn, (const uint8_t *)y->gate_w, y->gate_s, NULL,
                            (const uint8_t *)y->up_w, y->up_s, NULL, d->h, d->I, H, d->gs);
        else
            orc_swiglu_h_w8(d->xn, (const int8_t *)y->gate_w, y->gate_s, d->I, NULL,
                            (const int8_t *)y->up_w, y->up_s, d->I, NULL, d->h, d->I, H);
        if (d->wkind == 4)
            proj4(d, d->h, (const uint8_t *)y->down_w, y->down_s, d->use_v2 ? y->down_w2 : NULL,
                  NULL, d->dn, H, d->I);
        else
            proj(d, d->wkind, d->h, y->down_w, y->down_s, NULL, d->dn, H, d->I);
        for (int64_t i = 0; i < H; ++i) d->x[i] += d->dn[i];
    }
    if (d->layer_path)
        orc_rms_norm_torch(d->x, d->final_norm, d->xn, H, d->eps);
    else
        orc_rms_norm(d->x, d->final_norm, d->xn, H, d->eps);
    if (d->lmkind == 4)
        proj4(d, d->xn, (const uint8_t *)d->lm_w, d->lm_s, d->lm_w2, NULL, d->logits, d->V, H);
    else
        proj(d, d->lmkind, d->xn, d->lm_w, d->lm_s, NULL, d->logits, d->V, H);
}

/* Copy a prefilled KV prefix, decoder.rs:479-523: src is [hkv, src_max, hd]. */
ORC_API int orc_decoder_copy_kv(orc_decoder *d, int64_t l, const float *k, const float *v,
                                int64_t src_max, int64_t seq_len) {
    if (l < 0 || l >= d->L || seq_len > d->max_seq || seq_len > src_max) return -1;
    float *kc = orc_decoder_k_cache(d, l), *vc = orc_decoder_v_cache(d, l);
    for (int64_t h = 0; h < d->hkv; ++h)
        for (int64_t t = 0; t < seq_len; ++t) {
            memcpy(kc + (h * d->max_seq + t) * d->hd, k + (h * src_max + t) * d->hd,
                   (size_t)d->hd * 4);
            memcpy(vc + (h * d->max_seq + t) * d->hd, v + (h * src_max + t) * d->hd,
                   (size_t)d->hd * 4);
        }
    if (seq_len > d->kv_used) d->kv_used = seq_len;
    return 0;
}

ORC_API void orc_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

ORC_API int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

// Device helpers shared by the GEMV kernels (INT4 w4_gemv.hip, INT8/FP32
// gemv_dense.hip) and the decoder kernels that produce GEMV inputs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "w4_gemv.hpp"

namespace tb {
namespace gemv {

constexpr int kMaxWaves = 8;   // 512 threads per block: 256 VGPRs per lane available

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int N>
struct Log2 {
    static constexpr int value = 1 + Log2<N / 2>::value;
};
template <>
struct Log2<1> {
    static constexpr int value = 0;
};

inline int ceil_log2(int v) {
    int b = 0;
    while ((1 << b) < v) ++b;
    return b;
}

// Streamed-once weights: non-temporal 128-bit loads keep them from displacing
// activations, scales and partials in L2 / Infinity Cache.
__device__ __forceinline__ u32x4 load_nt16(const void *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

// q & mask, opaque to the optimiser.  With the mask visible, the compiler folds
// "(float)((q & 0x0F0F0F0F) >> 8 & 0xFF)" into v_bfe_u32 + v_cvt_f32_ubyte0 (two
// instructions per byte); behind this AND each byte converts with a single
// v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ uint32_t and_opaque(uint32_t q, uint32_t mask) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(q), "v"(mask));
    return r;
}

__device__ __forceinline__ uint32_t xor_opaque(uint32_t q, uint32_t mask) {
    uint32_t r;
    asm("v_xor_b32 %0, %1, %2" : "=v"(r) : "v"(q), "v"(mask));
    return r;
}

// a if !pick_b else b, as bit operations: a plain `pick ? v[i + h] : v[i]` on a
// register array is rewritten by the compiler into a dynamically indexed
// access (a cmp/cndmask chain over the whole array).
__device__ __forceinline__ float select_bits(float a, float b, uint32_t mask_b) {
    return __uint_as_float((__float_as_uint(a) & ~mask_b) | (__float_as_uint(b) & mask_b));
}

// Reduce V per-lane values over the lanes of bits [0, b) of the lane id
// (halving exchanges through ds_bpermute: V - 1 exchanges for V values instead
// of log2(64) per value).  After the call, lane l holds in v[0] the full sum of
// value index (l >> (b - log2 V)) & (V - 1) over its 2^b-lane span.
// Requires V <= 2^b.
template <int V>
__device__ __forceinline__ void transpose_reduce(float (&v)[V], int lane, int b) {
    constexpr int LOGV = Log2<V>::value;
#pragma unroll
    for (int s = 0; s < LOGV; ++s) {
        const int h = (V >> s) >> 1;
        const int mask = 1 << (b - 1 - s);
        const uint32_t up = (lane & mask) ? 0xFFFFFFFFu : 0u;
#pragma unroll
        for (int i = 0; i < h; ++i) {
            const float lo = v[i], hi = v[i + h];
            const float keep = select_bits(lo, hi, up);
            const float send = select_bits(hi, lo, up);
            v[i] = keep + __shfl_xor(send, mask);
        }
    }
    for (int sh = b - LOGV - 1; sh >= 0; --sh) v[0] += __shfl_xor(v[0], 1 << sh);
}

// silu(g) = g / (1 + exp(-g)), as the reference writes it
// (src/quantization/fused_ops.rs:404-405).
__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// Lane layout of one GEMV block: `nwaves` K-slices of `sw` chunk-lanes; a row
// spans 2^b lanes and `rps` rows are processed side by side per step.
struct Layout {
    int c, sw, b, rps, rpb;   // chunks per row, lanes per slice, log2 span, rows/step, rows/block
    int nwaves;
};

// Picks the split of a row of `c` chunks over waves and lanes for V partials
// per lane.  Returns false when the row needs more than kMaxWaves slices.
inline bool make_layout(int c, int logv, int j, Layout &L) {
    int bnat;
    if (c <= 64) {
        L.nwaves = 1;
        bnat = ceil_log2(c);
        L.sw = c;
    } else {
        L.nwaves = (c + 63) / 64;
        bnat = 6;
        L.sw = (c + L.nwaves - 1) / L.nwaves;
    }
    if (L.nwaves > kMaxWaves) return false;
    L.c = c;
    L.b = bnat > logv ? bnat : logv;
    L.rps = 64 >> L.b;
    L.rpb = j * L.rps;
    return true;
}

// Rotation-pair order of the rows of a head: logical rows 2i and 2i+1 of head
// h are physical rows h*hd + i and h*hd + i + hd/2.
__device__ __forceinline__ int rope_row(int l, int hd) {
    const int head = l / hd, r = l - head * hd, i = r >> 1;
    return head * hd + ((r & 1) ? i + (hd >> 1) : i);
}

// Output side of a GEMV block.  Row scales (per-channel INT8) multiply the row
// dot before bias: y = dot * s + b, as the reference's w8a32 rows do
// (src/quantization/gemv.rs:777-785).
struct Epi {
    const float *b0, *b1;     // bias of the (first, second) matrix or null
    const float *rs0, *rs1;   // per-row scales or null; *_len == 1 -> one scalar
    int rs0_len, rs1_len;
    const float *res;         // residual [m, n] for EPI_RESID
    float *y;                 // output [m, n]
    int n, m;
    RopeArgs rope;            // EPI_ROPE (m == 1)
};

__device__ __forceinline__ float row_scale(const float *rs, int len, int row) {
    return rs ? (len > 1 ? rs[row] : rs[0]) : 1.0f;
}

// Cross-lane + cross-wave reduction of the V = D*J*M per-lane partials and the
// epilogue.  Value index of a partial: (d * J + j) * M + m.
template <int V, int J, int M, bool DUAL, int EPI>
__device__ __forceinline__ void reduce_and_store(float (&v)[V], float *red, const Layout &L,
                                                 int lane, int wave, int row0, const Epi &e) {
    constexpr int LOGV = Log2<V>::value;
    constexpr int OUT = J * M;
    const int rr = lane >> L.b;
    const int cl = lane & ((1 << L.b) - 1);
    transpose_reduce<V>(v, lane, L.b);
    const int low = L.b - LOGV;
    if ((cl & ((1 << low) - 1)) == 0) {
        const int idx = (cl >> low) & (V - 1);
        red[(wave * L.rps + rr) * V + idx] = v[0];
    }
    __syncthreads();
    const int t = threadIdx.x;
    if (t < L.rps * OUT) {
        const int r2 = t / OUT, jm = t - r2 * OUT;
        const int j = jm / M, m = jm - j * M;
        const int row = row0 + j * L.rps + r2;
        if (row < e.n && m < e.m) {
            float a0 = 0.f, a1 = 0.f;
            for (int w = 0; w < L.nwaves; ++w) {
                const float *rw = red + (w * L.rps + r2) * V;
                a0 += rw[j * M + m];
                if (DUAL) a1 += rw[(J + j) * M + m];
            }
            const size_t o = (size_t)m * e.n + row;
            if (EPI == EPI_ROPE) {
                // Both rows of the rotation pair are in this block: logical rows
                // lr and lr ^ 1 (RoPE: src/llm/decoder.rs:28-68, products
                // rounded separately; KV append: decoder.rs:1137-1146).
                const RopeArgs &R = e.rope;
                const int lr = row, pl = lr ^ 1;
                const int pj = (pl - row0) / L.rps, pr2 = (pl - row0) - pj * L.rps;
                float ap = 0.f;
                for (int w = 0; w < L.nwaves; ++w) ap += red[(w * L.rps + pr2) * V + pj * M];
                const int prow = rope_row(lr, R.hd), qrow = rope_row(pl, R.hd);
                const float own = a0 * row_scale(e.rs0, e.rs0_len, prow) + (e.b0 ? e.b0[prow] : 0.f);
                const float oth = ap * row_scale(e.rs0, e.rs0_len, qrow) + (e.b0 ? e.b0[qrow] : 0.f);
                const int head = prow / R.hd, r = prow - head * R.hd, half = R.hd >> 1;
                const int pos = *R.pos;
                float val = own;
                if (head < R.hq + R.hkv) {
                    const int i = r < half ? r : r - half;
                    const float c = R.cos_t[(size_t)pos * R.hd + r];
                    const float s = R.sin_t[(size_t)pos * R.hd + r];
                    // r < half: own = x1, oth = x2 -> x1*c - x2*s; else own = x2 -> x2*c + x1*s
                    val = r < half ? __fsub_rn(__fmul_rn(own, c), __fmul_rn(oth, s))
                                   : __fadd_rn(__fmul_rn(own, c), __fmul_rn(oth, s));
                    (void)i;
                }
                if (head < R.hq) {
                    e.y[prow] = val;
                } else if (head < R.hq + R.hkv) {
                    R.kc[((size_t)(head - R.hq) * R.max_seq + pos) * R.hd + r] = val;
                } else {
                    R.vc[((size_t)(head - R.hq - R.hkv) * R.max_seq + pos) * R.hd + r] = val;
                }
            } else if (EPI == EPI_SWIGLU) {
                const float g = a0 * row_scale(e.rs0, e.rs0_len, row) + (e.b0 ? e.b0[row] : 0.f);
                const float u = a1 * row_scale(e.rs1, e.rs1_len, row) + (e.b1 ? e.b1[row] : 0.f);
                e.y[o] = silu(g) * u;
            } else {
                const float val =
                    a0 * row_scale(e.rs0, e.rs0_len, row) + (e.b0 ? e.b0[row] : 0.f);
                e.y[o] = (EPI == EPI_RESID) ? e.res[o] + val : val;
            }
        }
    }
}

// Builds one x chunk record (kXRecDwords) cooperatively in a group of 8
// consecutive lanes; lane `sub` (0..7) holds elements 4*sub .. 4*sub + 3 of the
// 32-element chunk in v.  x_i ~= sx * X_i with sx = 2^(e - 23), amax < 2^e,
// |X_i| < 2^23: the power-of-two step makes the scaling exact and rounds off
// only bits below 2^(e - 23), the precision an f32 partial sum of this chunk
// has.  Limb l of U_i = X_i + 2^23 (bits [4l, 4l + 4)) goes to nibble (i & 7) of
// dword limb[l][i >> 3], the nibble order of the packed weights.  All 8 lanes
// must call this; `out` is written when `live`.
__device__ __forceinline__ void build_xrec8(float4 v, int sub, bool live, uint32_t *out) {
    const float xv[4] = {v.x, v.y, v.z, v.w};
    int fin = 1;
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        fin &= __builtin_isfinite(xv[i]) != 0;
        amax = fmaxf(amax, fabsf(xv[i]));
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, o));
        fin &= __shfl_xor(fin, o);
    }
    int e = 0;
    (void)frexpf(amax, &e);
    e = e < -100 ? -100 : e;
    const float inv = ldexpf(1.0f, 23 - e);
    uint32_t lw[6] = {0u, 0u, 0u, 0u, 0u, 0u};
    int ssum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int X = fin ? (int)rintf(xv[i] * inv) : 0;
        X = X > 8388607 ? 8388607 : (X < -8388607 ? -8388607 : X);
        ssum += X;
        const uint32_t U = (uint32_t)(X + 8388608);
        const int nib = (sub & 1) * 4 + i;   // nibble of element 4*sub + i in its dword
#pragma unroll
        for (int l = 0; l < 6; ++l) lw[l] |= ((U >> (4 * l)) & 15u) << (4 * nib);
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) ssum += __shfl_xor(ssum, o);
#pragma unroll
    for (int l = 0; l < 6; ++l) lw[l] |= __shfl_xor(lw[l], 1);
    if (!live) return;
    if ((sub & 1) == 0) {
#pragma unroll
        for (int l = 0; l < 6; ++l) out[l * 4 + (sub >> 1)] = lw[l];
    }
    if (sub == 0) {
        out[24] = __float_as_uint(fin ? ldexpf(1.0f, e - 23) : __builtin_nanf(""));
        out[25] = (uint32_t)ssum;
    }
}

}  // namespace gemv
}  // namespace tb

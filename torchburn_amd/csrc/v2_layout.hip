// The v2 INT4 layout and the W4A8 activation semantics, on gfx950.
//
// v2 (packed_v2.rs:26-143): each 64-element group of a row is one 34-byte
// block, 32 bytes of v1 nibbles then the group scale as little-endian IEEE
// binary16.  k_pack_v2 replaces pack_rows_w4a32_group64_v1_to_v2
// (packed_v2.rs:114-143) with f32_to_f16's round-to-nearest-even
// (packed_v2.rs:66-105); k_dequant_v2 replaces dequantize_int4_grouped_v2
// (python/torchburn/quantization.py:155-169).  The GEMV over the blocks is the
// V2 form of k_w4_gemv / k_w4_mfma.
//
// W4A8 (gemv.rs:1353-1389): on hosts with AVX-512 VNNI the reference's group-64
// GEMVs first quantize each activation row to bytes, s_x = max(max|x|, 1e-10) /
// 127, q = round-to-nearest-even(x * (1 / s_x)), and contract q exactly with the
// nibbles.  k_act_u8 writes x' = q * s_x per row; a GEMV over x' reproduces
// that result to f32 rounding.
#include <math.h>

#include "gemv_common.hpp"
#include "tb_common.hpp"
#include "v2_layout.hpp"

namespace tb {

using namespace gemv;

namespace {

// binary32 -> binary16 bits, round to nearest even, in integer arithmetic:
// NaN -> sign | 0x7E00, overflow -> +-inf, below half the smallest subnormal
// -> +-0 (packed_v2.rs:66-105).
__device__ __forceinline__ uint32_t f32_to_f16_bits(float v) {
    const uint32_t x = __float_as_uint(v);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int e = (int)((x >> 23) & 0xFFu);
    const uint32_t m = x & 0x7FFFFFu;
    if (e == 0xFF) return sign | (m ? 0x7E00u : 0x7C00u);
    const int ub = e - 127;
    if (ub > 15) return sign | 0x7C00u;
    if (ub < -25) return sign;
    const bool normal = ub >= -14;
    const uint32_t sig = normal ? m : (m | 0x800000u);
    const uint32_t drop = normal ? 13u : (uint32_t)(-ub - 1);   // 13 .. 24
    const uint32_t base = normal ? (uint32_t)(ub + 15) << 10 : 0u;
    const uint32_t keep = sig >> drop, rem = sig & ((1u << drop) - 1u), half = 1u << (drop - 1u);
    uint32_t r = base + keep;   // a carry into the exponent is still RNE
    if (rem > half || (rem == half && (keep & 1u))) r += 1u;
    return sign | r;
}

// One thread per (row, group): 32 nibble bytes and the f16 scale into a
// 34-byte block (2-byte aligned: 17 half-word stores).
__global__ __launch_bounds__(256) void k_pack_v2(const uint8_t *__restrict__ w,
                                                 const float *__restrict__ s,
                                                 uint8_t *__restrict__ out, int64_t n, int ng) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n * ng) return;
    const int64_t row = t / ng;
    const int g = (int)(t - row * ng);
    const uint4 *src = reinterpret_cast<const uint4 *>(w + row * (int64_t)ng * 32 + g * 32);
    const uint4 a = src[0], b = src[1];
    const uint32_t d[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint16_t *dst = reinterpret_cast<uint16_t *>(out + t * kV2Block);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        dst[2 * i] = (uint16_t)(d[i] & 0xFFFFu);
        dst[2 * i + 1] = (uint16_t)(d[i] >> 16);
    }
    dst[16] = (uint16_t)f32_to_f16_bits(s[t]);
}

// s[i] = f16_to_f32(f32_to_f16(s[i])): scales as the v2 blocks carry them.
__global__ __launch_bounds__(256) void k_round_f16(float *__restrict__ s, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) s[i] = f16_bits_to_f32(f32_to_f16_bits(s[i]));
}

// One thread per (row, 32-element half block): (nib - 8) * f16 scale.
__global__ __launch_bounds__(256) void k_dequant_v2(const uint8_t *__restrict__ blocked,
                                                    float *__restrict__ out, int64_t n, int ng) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n * ng * 2) return;
    const int64_t blk = t >> 1;
    const int h = (int)(t & 1);
    const uint32_t o = (uint32_t)(blk * kV2Block);
    const u32x4 q = load_v2_chunk(blocked, o + 16u * (uint32_t)h);
    const float sc = load_v2_scale(blocked, o);
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
    float4 *dst = reinterpret_cast<float4 *>(out + t * 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (float)((int)((d[i] >> (4 * e)) & 15u) - 8) * sc;
        dst[2 * i] = make_float4(v[0], v[1], v[2], v[3]);
        dst[2 * i + 1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

// One block per activation row: s_x = max(max|x|, 1e-10) / 127, then
// x' = q * s_x with q = rint(x * (1 / s_x)) for the first 16 * (k / 16)
// elements and, as the reference's scalar tail does (gemv.rs:1383-1386),
// q = round-half-away(x / s_x) clamped to +-127 for the rest.  A NaN element
// gives q = 0 (the reference's int conversion of NaN lands on byte 128, i.e.
// q = 0); fmaxf skips NaN in the maximum.
// s_x of one row: max(max|x|, 1e-10) / 127 (a 256-thread block).
__device__ __forceinline__ float act_step(const float *xr, int k, float *red) {
    float mx = 0.f;
    for (int i = threadIdx.x; i < k; i += blockDim.x) mx = fmaxf(mx, fabsf(xr[i]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    if (mx < 1e-10f) mx = 1e-10f;
    return __fdiv_rn(mx, 127.0f);
}

// x' = q * s_x of element i of a row of k (body: the first 16 * (k / 16)).
__device__ __forceinline__ float act_elem(float v, int i, int body, float sx, float inv) {
    float q;
    if (i < body) {
        q = __builtin_rintf(__fmul_rn(v, inv));
    } else {
        q = fminf(fmaxf(roundf(__fdiv_rn(v, sx)), -127.f), 127.f);
    }
    return __fmul_rn(__builtin_isnan(q) ? 0.f : q, sx);
}

__global__ __launch_bounds__(256) void k_act_u8(const float *__restrict__ x,
                                                float *__restrict__ xo, int k) {
    __shared__ float red[4];
    const float *xr = x + (size_t)blockIdx.x * k;
    float *yr = xo + (size_t)blockIdx.x * k;
    const float sx = act_step(xr, k, red);
    const float inv = __fdiv_rn(1.0f, sx);
    const int body = k / 16 * 16;
    for (int i = threadIdx.x; i < k; i += blockDim.x) yr[i] = act_elem(xr[i], i, body, sx, inv);
}

// k_act_u8 that also writes the chunk records of x' (k % 32 == 0): eight lanes
// per 32-element chunk, each with one float4 of x, so the GEMV input of a
// W4A8 projection costs one pass instead of two.
__global__ __launch_bounds__(256) void k_act_rec(const float *__restrict__ x,
                                                 float *__restrict__ xo,
                                                 uint32_t *__restrict__ xq, int k) {
    __shared__ float red[4];
    const float *xr = x + (size_t)blockIdx.x * k;
    float *yr = xo + (size_t)blockIdx.x * k;
    const int nc = k / 32;
    uint32_t *qr = xq + (size_t)blockIdx.x * nc * kXRecDwords;
    const float sx = act_step(xr, k, red);
    const float inv = __fdiv_rn(1.0f, sx);
    const int body = k / 16 * 16, n4 = k / 4;
    // every thread runs the same number of rounds: the record build's quad
    // exchanges need whole 8-lane groups
    for (int e0 = 0; e0 < n4; e0 += blockDim.x) {
        const int e = e0 + (int)threadIdx.x;
        const bool live = e < n4;   // k % 32 == 0: whole 8-lane groups are live or not
        float4 v = live ? reinterpret_cast<const float4 *>(xr)[e] : make_float4(0.f, 0.f, 0.f, 0.f);
        v.x = act_elem(v.x, 4 * e, body, sx, inv);
        v.y = act_elem(v.y, 4 * e + 1, body, sx, inv);
        v.z = act_elem(v.z, 4 * e + 2, body, sx, inv);
        v.w = act_elem(v.w, 4 * e + 3, body, sx, inv);
        if (live) reinterpret_cast<float4 *>(yr)[e] = v;
        build_xrec8(v, e & 7, live, qr, nc, live ? e >> 3 : 0);
    }
}

}  // namespace

int pack_v1_to_v2(const uint8_t *w, const float *s, uint8_t *out, int64_t n, int64_t k,
                  hipStream_t st) {
    const int ng = (int)(k / 64);
    const int64_t total = n * ng;
    if (total == 0) return TB_OK;
    hipLaunchKernelGGL(k_pack_v2, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, w, s,
                       out, n, ng);
    TB_LAUNCHED();
    return TB_OK;
}

int dequant_v2(const uint8_t *blocked, float *out, int64_t n, int64_t k, hipStream_t st) {
    const int ng = (int)(k / 64);
    const int64_t total = n * ng * 2;
    if (total == 0) return TB_OK;
    hipLaunchKernelGGL(k_dequant_v2, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                       blocked, out, n, ng);
    TB_LAUNCHED();
    return TB_OK;
}

int round_scales_f16(float *s, int64_t n, hipStream_t st) {
    if (n == 0) return TB_OK;
    hipLaunchKernelGGL(k_round_f16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, s, n);
    TB_LAUNCHED();
    return TB_OK;
}

int act_u8(const float *x, float *xo, int64_t m, int64_t k, hipStream_t st) {
    if (m == 0) return TB_OK;
    hipLaunchKernelGGL(k_act_u8, dim3((unsigned)m), dim3(256), 0, st, x, xo, (int)k);
    TB_LAUNCHED();
    return TB_OK;
}

int act_rec(const float *x, float *xo, uint32_t *xq, int64_t m, int64_t k, hipStream_t st) {
    TB_REQUIRE(k % 32 == 0, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: W4A8 records need K % 32 == 0");
    if (m == 0) return TB_OK;
    hipLaunchKernelGGL(k_act_rec, dim3((unsigned)m), dim3(256), 0, st, x, xo, xq, (int)k);
    TB_LAUNCHED();
    return TB_OK;
}

}  // namespace tb

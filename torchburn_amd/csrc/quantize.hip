// Weight quantizers on gfx950: the formats the GEMVs read, produced on the
// device straight from f32 checkpoint tensors.
//
//   * grouped INT4 (python/torchburn/quantization.py:53-118): per group of
//     group_size elements s = max(max|w| / 7, 1e-8), q = clamp(
//     round_half_even(w / s), -8, 7), byte j = (q[2j] + 8) | (q[2j+1] + 8) << 4.
//     Groups of 32 or 64: one wavefront per 64-element span of a row, lane e
//     holds element e and the group maximum is a butterfly over the group's
//     lanes.  Any other group size: one wavefront per group for the scales,
//     then one thread per byte (its two elements may lie in two groups).
//   * per-channel INT8 (src/quantization/fused_ops.rs:554-589): s = max|w| / 127
//     (1 when max|w| <= 1e-8), q = clamp(round_half_away(w * (1 / s)), -127, 127).
//     One block per row.
//   * per-channel INT4 (quantize_linear_weights_int4, src/quantization/fused_ops.rs:
//     592-639): s = max|w| / 7 (1 when max|w| <= 1e-8), q = clamp(round_half_away(
//     w * (1 / s)), -8, 7) + 8 packed two per byte; an odd K pads its last byte
//     with the nibble 8.  One block per row.
//   * v2 -> v1 (python/torchburn/llm/loader.py:540-561, the cache migration):
//     32 nibble bytes copied, the binary16 scale widened to f32.
#include <math.h>

#include <algorithm>

#include "gemv_common.hpp"
#include "quantize.hpp"
#include "tb_common.hpp"

namespace tb {

using namespace gemv;

namespace {

template <int GS>
__global__ __launch_bounds__(256) void k_quant_int4(const float *__restrict__ w,
                                                    uint8_t *__restrict__ packed,
                                                    float *__restrict__ scales, int64_t n, int k) {
    const int lane = threadIdx.x & 63;
    const int spans = (k + 63) / 64;
    const int64_t span = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (span >= n * spans) return;   // whole waves leave together
    const int64_t row = span / spans;
    const int c0 = (int)(span - row * spans) * 64;
    const bool valid = c0 + lane < k;
    const float v = valid ? w[row * k + c0 + lane] : 0.f;
    float amax = fabsf(v);
#pragma unroll
    for (int off = 1; off < GS; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float s = fmaxf(__fdiv_rn(amax, 7.0f), 1e-8f);
    float q = __builtin_rintf(__fdiv_rn(v, s));
    q = fminf(fmaxf(q, -8.0f), 7.0f);
    const uint32_t u = (uint32_t)((int)q + 8);
    const uint32_t hi = (uint32_t)__shfl_down((int)u, 1);
    if (valid && (lane & 1) == 0)
        packed[row * (k / 2) + (c0 + lane) / 2] = (uint8_t)(u | (hi << 4));
    if (valid && (lane % GS) == 0) scales[row * (k / GS) + (c0 + lane) / GS] = s;
}

// Any group size: the scale of group id (row id / (k / gs)), one wavefront each.
__global__ __launch_bounds__(256) void k_quant_int4_scales(const float *__restrict__ w,
                                                           float *__restrict__ scales, int64_t n,
                                                           int k, int gs) {
    const int lane = threadIdx.x & 63;
    const int64_t ng = k / gs;
    for (int64_t id = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); id < n * ng;
         id += (int64_t)gridDim.x * 4) {   // wave-uniform trip count
        const int64_t row = id / ng;
        const float *p = w + row * k + (id - row * ng) * gs;
        float amax = 0.f;
        for (int e = lane; e < gs; e += 64) amax = fmaxf(amax, fabsf(p[e]));
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
        if (lane == 0) scales[id] = fmaxf(__fdiv_rn(amax, 7.0f), 1e-8f);
    }
}

// Any group size: byte j of a row from elements 2 j and 2 j + 1 and their
// groups' scales.
__global__ __launch_bounds__(256) void k_quant_int4_pack(const float *__restrict__ w,
                                                         const float *__restrict__ scales,
                                                         uint8_t *__restrict__ packed, int64_t n,
                                                         int k, int gs) {
    const int64_t bpr = k / 2;
    for (int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x; id < n * bpr;
         id += (int64_t)gridDim.x * 256) {
        const int64_t row = id / bpr;
        const int e = 2 * (int)(id - row * bpr);
        const float *wr = w + row * k;
        const float *sr = scales + row * (k / gs);
        auto nib = [&](int c) {
            float q = __builtin_rintf(__fdiv_rn(wr[c], sr[c / gs]));
            q = fminf(fmaxf(q, -8.0f), 7.0f);
            return (uint32_t)((int)q + 8);
        };
        packed[id] = (uint8_t)(nib(e) | (nib(e + 1) << 4));
    }
}

__global__ __launch_bounds__(256) void k_quant_int8(const float *__restrict__ w,
                                                    int8_t *__restrict__ q,
                                                    float *__restrict__ scales, int k) {
    __shared__ float red[4];
    const float *wr = w + (size_t)blockIdx.x * k;
    float mx = 0.f;
    for (int i = threadIdx.x; i < k; i += blockDim.x) mx = fmaxf(mx, fabsf(wr[i]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = mx > 1e-8f ? __fdiv_rn(mx, 127.0f) : 1.0f;
    const float inv = __fdiv_rn(1.0f, s);
    if (threadIdx.x == 0) scales[blockIdx.x] = s;
    int8_t *qr = q + (size_t)blockIdx.x * k;
    for (int i = threadIdx.x; i < k; i += blockDim.x) {
        const float t = __fmul_rn(wr[i], inv);
        qr[i] = (int8_t)fminf(fmaxf(roundf(t), -127.0f), 127.0f);   // roundf: ties away
    }
}

__global__ __launch_bounds__(256) void k_quant_int4_rows(const float *__restrict__ w,
                                                         uint8_t *__restrict__ packed,
                                                         float *__restrict__ scales, int k) {
    __shared__ float red[4];
    const float *wr = w + (size_t)blockIdx.x * k;
    float mx = 0.f;
    for (int i = threadIdx.x; i < k; i += blockDim.x) mx = fmaxf(mx, fabsf(wr[i]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = mx > 1e-8f ? __fdiv_rn(mx, 7.0f) : 1.0f;
    const float inv = __fdiv_rn(1.0f, s);
    if (threadIdx.x == 0) scales[blockIdx.x] = s;
    const int kp = (k + 1) / 2;
    uint8_t *pr = packed + (size_t)blockIdx.x * kp;
    for (int j = threadIdx.x; j < kp; j += blockDim.x) {
        uint32_t nib[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int e = 2 * j + h;
            // roundf: ties away from zero, as Rust's f32::round; a NaN (a NaN
            // weight, or an infinite one times inv = 0) stays NaN through
            // Rust's clamp and casts to 0, so its nibble is 8
            const float t = e < k ? roundf(__fmul_rn(wr[e], inv)) : 0.f;
            const float q = __builtin_isnan(t) ? 0.f : fminf(fmaxf(t, -8.0f), 7.0f);
            nib[h] = (uint32_t)((int)q + 8) & 15u;
        }
        pr[j] = (uint8_t)(nib[0] | (nib[1] << 4));
    }
}

// One thread per block: 32 nibble bytes, then the f16 scale as f32.
__global__ __launch_bounds__(256) void k_unpack_v2(const uint8_t *__restrict__ blocked,
                                                   uint8_t *__restrict__ w,
                                                   float *__restrict__ s, int64_t total) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const uint32_t o = (uint32_t)(t * kV2Block);
    const u32x4 a = load_v2_chunk(blocked, o), b = load_v2_chunk(blocked, o + 16u);
    uint4 *dst = reinterpret_cast<uint4 *>(w + t * 32);
    dst[0] = make_uint4(a.x, a.y, a.z, a.w);
    dst[1] = make_uint4(b.x, b.y, b.z, b.w);
    s[t] = load_v2_scale(blocked, o);
}

}  // namespace

int quantize_int4_grouped(const float *w, uint8_t *packed, float *scales, int64_t n, int64_t k,
                          int gs, hipStream_t st) {
    if (gs != 32 && gs != 64) {
        const int64_t groups = n * (k / gs), bytes = n * (k / 2);
        if (groups == 0) return TB_OK;
        // grid-stride loops: at most 65536 blocks of each
        hipLaunchKernelGGL(k_quant_int4_scales,
                           dim3((unsigned)std::min<int64_t>((groups + 3) / 4, 65536)), dim3(256),
                           0, st, w, scales, n, (int)k, gs);
        TB_LAUNCHED();
        if (bytes == 0) return TB_OK;
        hipLaunchKernelGGL(k_quant_int4_pack,
                           dim3((unsigned)std::min<int64_t>((bytes + 255) / 256, 65536)),
                           dim3(256), 0, st, w, scales, packed, n, (int)k, gs);
        TB_LAUNCHED();
        return TB_OK;
    }
    const int64_t waves = n * ((k + 63) / 64);
    if (waves == 0) return TB_OK;
    const dim3 grid((unsigned)((waves + 3) / 4));
    if (gs == 32)
        hipLaunchKernelGGL(k_quant_int4<32>, grid, dim3(256), 0, st, w, packed, scales, n, (int)k);
    else
        hipLaunchKernelGGL(k_quant_int4<64>, grid, dim3(256), 0, st, w, packed, scales, n, (int)k);
    TB_LAUNCHED();
    return TB_OK;
}

int quantize_int4_rows(const float *w, uint8_t *packed, float *scales, int64_t n, int64_t k,
                       hipStream_t st) {
    if (n == 0) return TB_OK;
    hipLaunchKernelGGL(k_quant_int4_rows, dim3((unsigned)n), dim3(256), 0, st, w, packed, scales,
                       (int)k);
    TB_LAUNCHED();
    return TB_OK;
}

int quantize_int8(const float *w, int8_t *q, float *scales, int64_t n, int64_t k,
                  hipStream_t st) {
    if (n == 0) return TB_OK;
    hipLaunchKernelGGL(k_quant_int8, dim3((unsigned)n), dim3(256), 0, st, w, q, scales, (int)k);
    TB_LAUNCHED();
    return TB_OK;
}

int unpack_v2_to_v1(const uint8_t *blocked, uint8_t *w, float *s, int64_t n, int64_t k,
                    hipStream_t st) {
    const int64_t total = n * (k / 64);
    if (total == 0) return TB_OK;
    hipLaunchKernelGGL(k_unpack_v2, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                       blocked, w, s, total);
    TB_LAUNCHED();
    return TB_OK;
}

}  // namespace tb

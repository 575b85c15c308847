// Any-shape INT4 / INT8 GEMV for gfx950: the fallback of the stateless
// projections for shapes the streaming kernels (w4_gemv.hip, gemv_dense.hip)
// do not take -- K not a multiple of 32 (the reference handles tail groups and
// odd K, src/quantization/gemv.rs:1650-1660, 1486-1502), group sizes that are
// not powers of two, and K past the streaming kernels' split-K range.
//
// One wavefront per (output row, activation row).  For INT4 the lanes walk the
// row's bytes (element 2j in the low nibble, 2j+1 in the high one, each q + 8;
// python/torchburn/quantization.py:89-94); a row of odd K ends in a half-used
// byte.  Grouped scales accumulate per element as s_g * (q * x); per-row and
// per-tensor scales multiply the row dot, y = dot * s + b (w4a32_linear,
// gemv.rs:1066-1182; gemv_w8a32, gemv.rs:777-785).  The wave sum is a butterfly.
#include "gemv_common.hpp"
#include "gemv_generic.hpp"
#include "tb_common.hpp"

namespace tb {

using namespace gemv;

namespace {

__device__ __forceinline__ float row_dot(const GenericParams &p, const void *wv, const float *s,
                                         int mode, int64_t row, const float *x, int lane) {
    float acc = 0.f;
    if (p.bits == 4) {
        const int64_t bpr = (p.k + 1) / 2;
        const uint8_t *w = static_cast<const uint8_t *>(wv) + row * bpr;
        const int64_t ng = (p.k + p.group - 1) / p.group;
        const float *sr = s + row * ng;
        for (int64_t j = lane; j < bpr; j += 64) {
            const uint32_t b = w[j];
            const int64_t e0 = 2 * j, e1 = e0 + 1;
            const float q0 = (float)((int)(b & 15u) - 8), q1 = (float)((int)(b >> 4) - 8);
            const float t0 = q0 * x[e0];
            const float t1 = e1 < p.k ? q1 * x[e1] : 0.f;
            if (mode == 0) {
                acc = fmaf(t0, sr[e0 / p.group], acc);
                if (e1 < p.k) acc = fmaf(t1, sr[e1 / p.group], acc);
            } else {
                acc += t0 + t1;
            }
        }
    } else {
        const int8_t *w = static_cast<const int8_t *>(wv) + row * p.k;
        for (int64_t j = lane; j < p.k; j += 64) acc = fmaf((float)w[j], x[j], acc);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
    if (mode == 1) acc *= s[row];
    if (mode == 2) acc *= s[0];
    return acc;
}

__global__ __launch_bounds__(256) void k_gemv_generic(GenericParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t m = blockIdx.y;
    if (row >= p.n) return;   // whole waves leave together
    const float *x = p.x + m * p.k;
    float a = row_dot(p, p.w0, p.s0, p.scale_mode0, row, x, lane) + (p.b0 ? p.b0[row] : 0.f);
    if (p.w1) {
        const float u =
            row_dot(p, p.w1, p.s1, p.scale_mode1, row, x, lane) + (p.b1 ? p.b1[row] : 0.f);
        a = silu(a) * u;
    } else if (p.res) {
        a = p.res[m * p.n + row] + a;
    }
    if (lane == 0) p.y[m * p.n + row] = a;
}

}  // namespace

int gemv_generic(const GenericParams &p, hipStream_t st) {
    if (p.m == 0 || p.n == 0) return TB_OK;
    TB_REQUIRE(p.m < 65536 && p.n < (1ll << 33), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: generic GEMV: too many rows");
    TB_REQUIRE(p.bits == 8 || p.group > 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: generic GEMV: group size must be positive");
    const dim3 grid((unsigned)((p.n + 3) / 4), (unsigned)p.m);
    hipLaunchKernelGGL(k_gemv_generic, grid, dim3(256), 0, st, p);
    TB_LAUNCHED();
    return TB_OK;
}

}  // namespace tb

// Internal launcher of the any-shape GEMV (gemv_generic.hip): the shapes the
// streaming kernels do not take (K not a multiple of 32, group sizes that are
// not powers of two, K beyond the streaming kernels' split-K range).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tb {

struct GenericParams {
    const float *x;       // [m, k]
    const void *w0;       // INT4: packed nibbles [n, ceil(k/2)]; INT8: [n, k]
    const float *s0;      // scales (layout by scale_mode)
    const float *b0;      // [n] or null
    const void *w1;       // SwiGLU pair: up projection, or null
    const float *s1;
    const float *b1;
    const float *res;     // [m, n] residual or null
    float *y;             // [m, n] (may alias res)
    int64_t m, n, k;
    int64_t group;        // INT4 grouped: elements per group (the last one may be short)
    // Scale layout: 0 = INT4 grouped [n, ceil(k/group)] applied per group;
    // 1 = one per row [n]; 2 = one per-tensor scalar [1] (modes 1 / 2 multiply the
    // row dot: y = dot * s + b).
    int scale_mode0, scale_mode1;
    int bits;             // 4 or 8
};

// y = epilogue(x . W^T): bias, optional residual, or silu(g) * u when w1 is set.
int gemv_generic(const GenericParams &p, hipStream_t st);

}  // namespace tb

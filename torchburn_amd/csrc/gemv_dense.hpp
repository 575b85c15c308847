// Internal launcher of the INT8 per-channel / FP32 GEMV kernels (gemv_dense.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "w4_gemv.hpp"

namespace tb {

enum WeightType { W_I8 = 8, W_F32 = 32 };

struct DenseParams {
    const float *x;     // [m, k] activations
    const void *w0;     // [n, k] int8 or f32 (gate when dual)
    const float *rs0;   // int8: per-row scales [n] (or [1]); f32: null
    int rs0_len;
    const float *b0;    // [n] bias or null
    const void *w1;     // up projection of a SwiGLU pair, or null
    const float *rs1;
    int rs1_len;
    const float *b1;
    const float *res;   // [m, n] residual for EPI_RESID
    float *y;           // [m, n]
    int m, n, k;
    RopeArgs rope;      // EPI_ROPE only
};

// One pass over m <= kMaxRowsPerPass activation rows; shapes validated by the
// caller except K % 32.
int dense_gemv(const DenseParams &p, int wt, int epi, hipStream_t st);

}  // namespace tb

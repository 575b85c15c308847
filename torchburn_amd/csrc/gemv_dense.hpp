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
    // Fused RMSNorm (M == 1), as W4Params.  Consumer: x holds x * w_norm and
    // ssq_in [ssq_n] the sums of squares of x over 16-element pieces; the row
    // dots are scaled by 1 / sqrt(sum / norm_h + eps) before the row scale.
    // Producer (INT8 only; 16-row blocks): y * rec_w in f32 into xw_out and the
    // 16-row sums of squares of y into ssq_out.
    const float *ssq_in;
    int ssq_n, norm_h;
    float eps;
    const float *rec_w;
    float *xw_out;
    float *ssq_out;
};

// One pass over m <= kMaxRowsPerPass activation rows; shapes validated by the
// caller except K % 32.
int dense_gemv(const DenseParams &p, int wt, int epi, hipStream_t st);

}  // namespace tb

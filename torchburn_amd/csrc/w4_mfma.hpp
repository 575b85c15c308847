// Internal launcher of the batched INT4 projection on FP32 MFMA (w4_mfma.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tb {

struct MfmaParams {
    const float *x;      // [m, k] activations
    const uint8_t *w0;   // [n, k/2] packed nibbles (gate when dual)
    const float *s0;     // [n, k/group] scales
    const float *b0;     // [n] bias or null
    const uint8_t *w1;   // up projection of a SwiGLU pair, or null
    const float *s1;
    const float *b1;
    const float *res;    // [m, n] residual (EPI_RESID)
    float *y;            // [m, n]
    int m, n, k;
    int gshift;          // log2(group_size)
    int scale_mode;      // 0: grouped [n, k/group]; 1: one scale per row; 2: one scalar
    int v2;              // 1: w0 / w1 are v2 streams of 34-byte group-64 blocks
                         // (f16 scales inside, s0 / s1 unused)
};

// Bytes of split-K partials w4_mfma needs for this shape (dual = SwiGLU pair).
size_t w4_mfma_partials_bytes(int m, int n, int k, bool dual);

// y = epilogue(x . deq(w)^T) for any m >= 1 (the MFMA tile is 16 rows; rows
// beyond m are padding).  epi: EPI_PLAIN, EPI_RESID, or EPI_SWIGLU when w1 is
// set.  part: device scratch of w4_mfma_partials_bytes().  Shapes validated by
// the caller (K % 32 == 0, K % group == 0, 16-byte aligned rows).
int w4_mfma(const MfmaParams &p, int epi, float *part, hipStream_t st);

}  // namespace tb

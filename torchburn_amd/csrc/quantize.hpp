// Internal launchers of the weight quantizers (quantize.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tb {

// f32 [n, k] -> v1 nibbles [n, k/2] + f32 scales [n, k/gs]; gs 32 or 64, k % gs == 0.
int quantize_int4_grouped(const float *w, uint8_t *packed, float *scales, int64_t n, int64_t k,
                          int gs, hipStream_t st);

// f32 [n, k] -> v1 nibbles [n, ceil(k/2)] + one f32 scale per row [n]
// (quantize_linear_weights_int4, fused_ops.rs:592-639).
int quantize_int4_rows(const float *w, uint8_t *packed, float *scales, int64_t n, int64_t k,
                       hipStream_t st);

// f32 [n, k] -> int8 [n, k] + per-row f32 scales [n].
int quantize_int8(const float *w, int8_t *q, float *scales, int64_t n, int64_t k,
                  hipStream_t st);

// v2 blocks [n, (k/64) * 34] -> v1 nibbles [n, k/2] (16-byte aligned) + f32 scales [n, k/64].
int unpack_v2_to_v1(const uint8_t *blocked, uint8_t *w, float *s, int64_t n, int64_t k,
                    hipStream_t st);

}  // namespace tb

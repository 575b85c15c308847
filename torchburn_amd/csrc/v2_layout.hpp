// Internal launchers of the v2-layout and W4A8 kernels (v2_layout.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tb {

// Bytes of one v2 block: 32 bytes of nibbles + the binary16 group scale.
constexpr int kV2Bytes = 34;

// v1 nibbles [n, k/2] (16-byte aligned) + f32 scales [n, k/64] -> v2 blocks
// [n, (k/64) * 34] with f16 scales (k % 64 == 0).
int pack_v1_to_v2(const uint8_t *w, const float *s, uint8_t *out, int64_t n, int64_t k,
                  hipStream_t st);

// v2 blocks [n, (k/64) * 34] (4-byte aligned) -> f32 weights [n, k] (16-byte aligned).
int dequant_v2(const uint8_t *blocked, float *out, int64_t n, int64_t k, hipStream_t st);

// Each f32 scale replaced by its binary16 rounding (RNE), in place.
int round_scales_f16(float *s, int64_t n, hipStream_t st);

// Per row of x [m, k]: x' = q * s_x, the activations the W4A8 tier contracts
// (the reference's byte rounding, gemv.rs:1353-1389: the first 16 * (k / 16)
// elements to nearest even, the rest half away from zero).
int act_u8(const float *x, float *xo, int64_t m, int64_t k, hipStream_t st);

// act_u8 plus the chunk records of x' into xq [m, 7, k/32, 4] (k % 32 == 0).
int act_rec(const float *x, float *xo, uint32_t *xq, int64_t m, int64_t k, hipStream_t st);

// The W4A8 semantics switch (tb_set_vnni_semantics).
bool vnni_semantics();

}  // namespace tb

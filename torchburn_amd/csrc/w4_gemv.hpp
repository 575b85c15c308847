// Internal launchers of the INT4 GEMV kernels (w4_gemv.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tb {

enum Epilogue { EPI_PLAIN = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_ROPE = 3 };

// EPI_ROPE: the QKV projection of a decoder step writes rotated q into y and
// the rotated k / plain v row of the current position into the KV cache.
// Output rows are visited in rotation-pair order (see rope_row) so each block
// holds both halves of every pair it rotates.
struct RopeArgs {
    const int *pos;           // device: current position
    const float *cos_t, *sin_t;   // cos / sin of position p at [p * tab_stride + i]
    float *kc, *vc;           // this layer's caches [hkv, max_seq, hd]
    int hq, hkv, hd, max_seq;
    int tab_stride;           // hd for [max_seq, hd] tables, 0 for one position's row
};

// Activation rows per GEMV pass (x is held in VGPRs).
constexpr int kMaxRowsPerPass = 2;     // INT8 / fp32 GEMV
constexpr int kMaxW4RowsPerPass = 4;   // INT4 GEMV

// An x chunk record: 32 activations as 24-bit fixed-point integers in six
// 4-bit limb planes (24 dwords), then {step of elements 0-15, step of 16-31,
// integer sum of 0-15, of 16-31} (steps as f32 bits, NaN when the half holds
// NaN/Inf): 112 bytes in 7 quads of 4 dwords.  A row's records are stored by
// quad (quad i of chunk c at (i * k/32 + c) * 4 dwords from the row's start),
// so a GEMV wave, one chunk per lane, reads each quad of 64 chunks as one
// contiguous KiB.  Built once per activation vector by xquant() or by the
// producing kernel, read by every block of the GEMV.
constexpr int kXRecDwords = 28;

struct W4Params {
    const float *x;    // [m, k] activations (read only by the NaN/Inf path)
    const uint32_t *xq; // [m, 7, k/32, 4] chunk records of x (xquant), by quad
    const uint8_t *w0; // [n, k/2] packed nibbles (gate when dual)
    const float *s0;   // [n, k/group] scales
    const float *b0;   // [n] bias or null
    const uint8_t *w1; // up projection of a SwiGLU pair, or null
    const float *s1;
    const float *b1;
    const float *res;  // [m, n] residual for EPI_RESID
    float *y;          // [m, n] output
    int m, n, k;
    int gshift;        // log2(group_size)
    int scale_mode;    // 0: grouped scales [n, k/group]; 1: one scale per row [n]
                       // (per-channel w4a32_linear); 2: one per-tensor scalar
    int v2;            // 1: w0 is the v2 stream of 34-byte group-64 blocks (f16
                       // scales inside, s0 unused; K % 64 == 0, 4-byte aligned)
    int rows_j;        // rows per block (tuning: 4, 8 or 16; 0 = default)
    RopeArgs rope;     // EPI_ROPE only
    // Fused RMSNorm (M == 1).  Consumer: xq holds records of x * w_norm (and
    // p.x that product in f32, for the NaN/Inf path); ssq_in [ssq_n] the sums
    // of squares of x over 16-element pieces; the dots are scaled by
    // 1 / sqrt(sum / norm_h + eps).
    const float *ssq_in;
    int ssq_n, norm_h;
    float eps;
    // Producer: y * rec_w as records into rec_out and in f32 into xw_out, and
    // the 16-row sums of squares of y into ssq_out (16-row blocks).
    uint32_t *rec_out;
    const float *rec_w;
    float *xw_out;
    float *ssq_out;
};

// One pass over m <= kMaxW4RowsPerPass activation rows.  Epilogue EPI_SWIGLU is implied when
// p.w1 is set.  Shapes are validated by the caller.
int w4_gemv(W4Params p, int epi, hipStream_t st);

// Chunk records of x [m, k] (k % 32 == 0) into xq [m, 7, k/32, 4] (by quad).
int xquant(const float *x, uint32_t *xq, int m, int k, hipStream_t st);

}  // namespace tb

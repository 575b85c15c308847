// Internal launchers of the small-batch INT4 projection on f16 MFMA
// (w4_limb.hip): up to 16 activation rows, every weight byte read once.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tb {

constexpr int kLimbMaxM = 16;

// Bytes of the activation records of an [m, k] batch (k % 128 == 0, m <= 16).
size_t limb_records_bytes(int m, int k);

struct LimbParams {
    const float *x;        // [m, k] activations (read by the f32 path of NaN / Inf groups)
    const uint8_t *rec;    // records of x (limb_prep)
    const uint8_t *w0;     // [n, k/2] v1 nibbles (gate when w1 is set)
    const float *s0;       // scales of w0: row stride scols, index kk >> gshift
    const float *b0;       // [n] bias or null
    const uint8_t *w1;     // up projection of a SwiGLU pair, or null
    const float *s1;
    const float *b1;
    const float *res;      // [m, n] residual or null (single projection)
    float *y;              // [m, n] output; silu(gate) * up for a pair
    uint8_t *rec_out;      // pair only: records of y for the next projection, or null
    int m, n, k;
    int scols;             // scales per row: k / group, 1 (per-row) or 0 (one scalar)
    int gshift;            // log2(group); 31 with per-row or scalar scales
};

// Bytes of split partials w4_limb needs (pair: SwiGLU gate + up).
size_t limb_partials_bytes(int m, int n, int k, bool pair);

// Records of x [m, k] (row stride k) into rec (limb_records_bytes(m, k)).
int limb_prep(const float *x, uint8_t *rec, int m, int k, hipStream_t st);

// Shapes the kernels take: 1 <= m <= 16, k % 128 == 0; a SwiGLU pair needs
// n % 128 == 0.  Pointers: x, w 16-byte aligned (checked by callers).
bool limb_shape_ok(int64_t m, int64_t n, int64_t k, bool pair);

// y = epilogue(x . deq(W)^T): plain / + bias / + residual for one projection,
// silu(x W0^T + b0) * (x W1^T + b1) for a pair (plus rec_out when set).
// part: device scratch of limb_partials_bytes().
int w4_limb(const LimbParams &p, float *part, hipStream_t st);

// Batched projection for larger M on the exact limbs (k_w4_lgemm): the FP32-MFMA
// kernel's tiling and split-K partial layout (w4_mfma.hip reduces them).
struct LGemmArgs {
    const float *x;         // [m, k] raw activations (the f32 path of flagged batches)
    const uint8_t *rec;     // lgemm_prep records: ceil(m / 16) slabs
    const uint8_t *w0;      // [n, k/2] nibbles (gate when dual)
    const float *s0;
    const uint8_t *w1;      // up projection of a SwiGLU pair, or null
    const float *s1;
    float *part;            // [dual + 1][splits][m][n] partials
    int m, n, k;
    int scols, gshift;      // scale of (row, kk) at s[row * scols + (kk >> gshift)]
    int klen, nbx, splits;  // K per split (a multiple of 128), 64-row blocks per matrix
    int batches, nslabs;    // k / 128, ceil(m / 16)
};
size_t lgemm_records_bytes(int m, int k);
int lgemm_prep(const float *x, uint8_t *rec, int m, int k, hipStream_t st);
// grid: (nbx * (dual + 1), splits, ceil(nslabs / mt)); mt slabs per block (1..4).
int lgemm_launch(const LGemmArgs &a, int mt, dim3 grid, hipStream_t st);

}  // namespace tb

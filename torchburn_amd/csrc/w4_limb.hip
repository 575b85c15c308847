// Small-batch grouped-INT4 projection Y[M, N] = X[M, K] . deq(W)^T for up to
// 16 activation rows on f16 MFMA (v_mfma_f32_16x16x32_f16), reading every
// weight byte once (the C ABI routes 3..16 rows here).
//
// Replaces the M > 1 path of the reference's w4a32_grouped_linear
// (src/quantization/packed_v2.rs:557-624 -> gemm_w4a32_grouped,
// src/quantization/gemv.rs:1690-1725), which runs one GEMV per activation row,
// and the batched MLP of fused_swiglu_mlp_batched_w4a32
// (src/quantization/fused_ops.rs:1267-1319) at decode-size batches.
//
// Arithmetic.  The contraction of one 32-element group is
//     sum_k (q_k - 8) x_k
// with q_k the stored nibble, computed exactly on the MFMA:
//   * weights: a nibble q placed in the low bits of an f16 is the subnormal
//     q * 2^-24 (nibbles at bits 4-7 of a byte give 16 q * 2^-24), so a dword
//     of 8 nibbles becomes 8 exact f16 operands with 4 ANDs and one shift;
//   * activations: each half batch of 64 elements of a row (2 groups) is
//     scaled by a power of two 2^e (its largest magnitude lands in
//     [2^14, 2^15)) and split into two fixed-point limbs on that grid: h1 a
//     multiple of 16 (|h1 / 16| <= 2048) and h2 a multiple of 2^-7
//     (|h2 2^7| <= 1024), both exact in f16, with |x 2^e - h1 - h2| <= 2^-8,
//     i.e. 2^-23 of the half batch's largest term;
//   * the -8 of every weight is one more MFMA of the limbs against a constant
//     B of -8 * 2^-24, shared by all weight rows, whose result is the C
//     operand of the weight MFMA.  Each limb has its own accumulation, so every
//     product and partial sum is an integer multiple of the limb's quantum below
//     2^21 quanta: the MFMA result is exact whatever the order and rounding of
//     its internal additions (they are not IEEE round-to-nearest, which a
//     float split of x would expose);
//   * per 32-element group the limb results are scaled by the weight row's
//     group scale and accumulated in f32; per half batch the sum is scaled by
//     2^(24 - e) into the running total.
// The error of a half batch's contribution is the limb quantization, ~2^-23
// of its largest term, the order of the f32 reference's own rounding.  A half
// batch holding NaN / Inf, or a largest magnitude outside [2^-100, 2^100], is
// flagged, and its batch runs an f32 MFMA path on the raw activations, so
// non-finite values propagate as in the reference's unpack-and-fma.
//
// Activation records (limb_prep, or the SwiGLU epilogue for the next
// projection), one per 128-element batch: for each of its 4 groups T f16 A
// tiles of 64 lanes x 16 bytes, then 32 bytes, byte 2 a + h for A-row a and
// half h (groups 2 h, 2 h + 1), holding the biased f32 exponent of
// 2^(24 - e), or 0 for a half that takes the f32 path (a valid exponent byte
// is never 0, so the flag travels with the record).  The two halves of a
// record may be written by different blocks.
//   * M <= 8 (T = 1): A-row i of the MFMA is limb (i >> 3) of row i & 7, so one
//     MFMA covers both limbs in separate output rows; the two limb halves of the
//     output are added at the end (lanes l and l + 32).
//   * 9 <= M <= 16 (T = 2): A-row i is row i; tile t is limb t (two MFMAs).
//   * Lane l (i = l % 16, k-slot q = l / 16) holds elements 8q + {0,4,1,5,2,6,
//     3,7} of the group (odd ones pre-divided by 16), the order in which
//     expand_nibbles unpacks a dword of nibbles.
//
// Work split.  The grid is (row chunks) x (K splits).  A block copies the
// records of its K range to LDS once (direct global-to-LDS loads, issued with
// the first weight loads so the block pays one memory latency), then each of
// its waves streams the weights of R 16-row blocks over that range: per batch
// a lane loads one 16-byte chunk per row block, lane (i, q) group g0 + q of
// row i, and a 4x4 transpose across the lane quarters (v_permlane32_swap,
// v_permlane16_swap) leaves dword q of group g0 + t in register t, the MFMA B
// operand layout.  Group scales come per quad of 4 batches, lane (i, q) the 4
// scales of batch q of row i in one 16-byte load, and reach the lanes of the
// row by ds_bpermute.  Weights and scales stream one quad ahead through a
// register ring; since the records come from LDS, each wait is for the oldest
// weights only (vector loads retire in order).  When the records of the whole
// K fit in LDS (M <= 8, K <= 4224) and the matrix has enough 16-row blocks,
// one block per CU covers the whole K with no split; for a SwiGLU pair that
// block holds the gate and up rows of 64 columns of h and writes h and its
// half of h's records itself.  Otherwise the per-split partial sums go to a
// scratch buffer and a small reduce kernel sums them in split order
// (deterministic) and runs the epilogue: bias (+ residual), or for a SwiGLU
// pair, whose gate and up rows are stacked as one 2n-row matrix,
// h = silu(g) * u plus the records of h for the next projection.
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "gemv_common.hpp"
#include "tb_common.hpp"
#include "w4_limb.hpp"

namespace tb {

using namespace gemv;

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kTile = 1024;          // one A tile: 64 lanes x 8 f16
constexpr int kBatch = 128;          // K per batch: one 16-byte chunk per lane
constexpr int kRecTail = 32;         // an exponent byte per A-row and half (0: the f32 path)
constexpr int kLdsBudget = 64 << 10; // records per block (two blocks per CU)
constexpr int kPairWaves = 8;        // the whole-K SwiGLU pair form
constexpr int kPairCols = 64;        // its columns of h per block: half a record batch

__host__ __device__ constexpr int tiles_of(int m) { return m <= 8 ? 1 : 2; }
// bytes of one batch record (4 groups)
__host__ __device__ constexpr int rec_stride(int tiles) { return 4 * tiles * kTile + kRecTail; }

// 8 nibbles of a dword -> the f16 B operand (subnormals q * 2^-24; the odd
// nibbles come out 16x larger, which their pre-divided activations undo).
// Slot order: n0, n4, 16 n1, 16 n5, n2, n6, 16 n3, 16 n7.
__device__ __forceinline__ h8 expand_nibbles(uint32_t d) {
    const uint32_t u = d >> 8;
    const u32x4 v = {d & 0x000F000Fu, d & 0x00F000F0u, u & 0x000F000Fu, u & 0x00F000F0u};
    return __builtin_bit_cast(h8, v);
}

// The B operand of the offset MFMA: -8 * 2^-24 in the slots of even elements,
// -128 * 2^-24 in those of the pre-divided odd ones (f16 subnormals).
__device__ __forceinline__ h8 offset_operand() {
    const u32x4 v = {0x80088008u, 0x80808080u, 0x80088008u, 0x80808080u};
    return __builtin_bit_cast(h8, v);
}

// Lane (i, q) holds dwords 0..3 of group g0 + q of its row; afterwards
// register t holds dword q of group g0 + t.  Transpose of 4 x 4 dwords across
// the lane quarters: v_permlane32_swap exchanges the upper half's first
// operand with the lower half's second, v_permlane16_swap the same between
// the 16-lane rows of each half.
__device__ __forceinline__ void transpose4(u32x4 &v) {
    const auto a = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
    const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    v.x = c[0]; v.y = c[1]; v.z = d[0]; v.w = d[1];
}

// The exponent of one half batch from each lane's largest magnitude mx and
// finiteness fin over its values (the whole wave holds the half): e places
// the largest magnitude in [2^14, 2^15); byte is the record's exponent byte,
// the biased f32 exponent of 2^(24 - e) (e in [-85, 115] -> [36, 236]), or 0
// when the half holds NaN / Inf or a magnitude outside [2^-100, 2^100].
struct HalfExp {
    int e;
    bool ok;   // this lane's values take the limbs
    uint8_t byte;
};
__device__ __forceinline__ HalfExp half_exp(float mx, bool fin) {
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    int E = 0;
    (void)frexpf(mx, &E);   // mx = f 2^E, f in [0.5, 1)
    const bool out_of_range = mx > 0.f && (E > 100 || E < -100);
    const bool bad = __any((!fin || out_of_range) ? 1 : 0) != 0;
    HalfExp r;
    r.e = (mx > 0.f && !out_of_range) ? 15 - E : 0;
    r.ok = fin && !out_of_range;
    r.byte = bad ? (uint8_t)0 : (uint8_t)(151 - r.e);
    return r;
}

// The two limbs of x in slot j of a lane's 8 (odd slots pairs hold the
// pre-divided odd elements).
__device__ __forceinline__ void limbs_of(float x, const HalfExp &he, int j, _Float16 &l1,
                                         _Float16 &l2) {
    const bool odd = ((j >> 1) & 1) != 0;
    const float xs = he.ok ? ldexpf(x, he.e) : 0.f;
    const float j1 = rintf(xs * 0.0625f);               // h1 = 16 j1
    const float j2 = rintf((xs - 16.0f * j1) * 128.0f);  // h2 = 2^-7 j2
    l1 = (_Float16)(odd ? j1 : 16.0f * j1);
    l2 = (_Float16)ldexpf(j2, odd ? -11 : -7);
}

// Element of the group held in slot j (the order expand_nibbles unpacks).
__host__ __device__ constexpr int slot_elem(int j) { return (j >> 1) | ((j & 1) << 2); }

// Half h of the record of one 128-element batch (groups 2 h, 2 h + 1), built
// by one wave.  Lane (i, q) holds v[g][e] = element 32 (2 h + g) + 8 q + e of
// the batch for its row (row i & 7 when T = 1, row i when T = 2; zeros beyond
// m).
template <int T>
__device__ void build_half(const float (&v)[2][8], int lane, uint8_t *rg, int h) {
    const int i = lane & 15, q = lane >> 4;
    float mx = 0.f;
    bool fin = true;
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            fin = fin && __builtin_isfinite(v[g][e]);
            mx = fmaxf(mx, fabsf(v[g][e]));
        }
    const HalfExp he = half_exp(mx, fin);
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        h8 l1, l2;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            _Float16 a, b;
            limbs_of(v[g][slot_elem(j)], he, j, a, b);
            l1[j] = a;
            l2[j] = b;
        }
        uint8_t *tg = rg + (size_t)(2 * h + g) * T * kTile;
        if (T == 1) {
            *reinterpret_cast<h8 *>(tg + lane * 16) = i < 8 ? l1 : l2;
        } else {
            *reinterpret_cast<h8 *>(tg + lane * 16) = l1;
            *reinterpret_cast<h8 *>(tg + kTile + lane * 16) = l2;
        }
    }
    if (q == 0) rg[4 * T * kTile + 2 * i + h] = he.byte;
}

// A batch whose record flags either half (exponent byte 0 for every A-row of
// a flagged half) runs the f32 path.
__device__ __forceinline__ bool flagged(const uint8_t *rg_tail) {
    const uint32_t v = *reinterpret_cast<const uint16_t *>(rg_tail);
    return (v & 0xFFu) == 0 || (v >> 8) == 0;
}

// One wave per half batch: lane (i, q) loads elements 32 (2 h + g) + 8 q ..
// of its row for the half's two groups g and builds that half of the record.
template <int T>
__device__ void limb_prep_body(const float *__restrict__ x, uint8_t *__restrict__ rec, int m,
                               int k, int batches) {
    const int lane = threadIdx.x & 63;
    const int hw = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (hw >= 2 * batches) return;   // whole waves
    const int b = hw >> 1, h = hw & 1;
    const int i = lane & 15, q = lane >> 4;
    const int row = T == 1 ? (i & 7) : i;
    float v[2][8];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        if (row < m) {
            const float *xp = x + (size_t)row * k + 128 * b + 32 * (2 * h + g) + 8 * q;
            const float4 a = *reinterpret_cast<const float4 *>(xp);
            const float4 c = *reinterpret_cast<const float4 *>(xp + 4);
            v[g][0] = a.x; v[g][1] = a.y; v[g][2] = a.z; v[g][3] = a.w;
            v[g][4] = c.x; v[g][5] = c.y; v[g][6] = c.z; v[g][7] = c.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[g][e] = 0.f;
        }
    }
    build_half<T>(v, lane, rec + (size_t)b * rec_stride(T), h);
}

// Partial sums of one block: rows [row0, row0 + 16 R NW) of the stacked
// weights (rows past n come from w1 / s1 for a SwiGLU pair) over the K range
// [ks, ks + ksl) of split blockIdx.y.  The records of that range are copied to
// LDS first (one pass, one barrier); the loop then waits only for weights.
// PE (a SwiGLU pair over the whole K, T = R = 1, NW = 8): block b takes
// columns [64 b, 64 b + 64) of h, wave w the gate (w even) or up (w odd) rows
// of its 16 columns 64 b + 16 (w / 2) ..; the block then writes h and half
// b % 2 of the record of h's batch b / 2 itself (no partials, no reduce).
template <int T, int R, int NW, int DQ, bool SV, bool PE>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2)))
void k_w4_limb(LimbParams p, float *__restrict__ part, int ksl, int ntot) {
    static_assert(!PE || (T == 1 && R == 1 && NW == 8), "the pair epilogue form");
    constexpr int BS = rec_stride(T);
    constexpr int ROWS = 16 * R * NW;
    extern __shared__ __align__(16) uint8_t lrec[];   // the (ksl / 128) batch records
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 15, q = lane >> 4;
    const int split = blockIdx.y;
    const int ks = split * ksl;
    const int ke = min(p.k, ks + ksl);
    const int b0 = ks / kBatch, nb = (ke - ks) / kBatch;
    const int klast = ke - kBatch;

    // the weight and scale rows of block row rl (rows past the stacked
    // [w0; w1] read row 0 and are never stored)
    auto row_ptrs = [&](int rl, const uint8_t *&w, const float *&sc) {
        const int row = blockIdx.x * ROWS + rl;
        bool second = row >= p.n && row < ntot;
        int rr = row < ntot ? (second ? row - p.n : row) : 0;
        if (PE) {   // rl = 16 wave + i
            second = (rl >> 4) & 1;
            rr = 64 * blockIdx.x + 16 * (rl >> 5) + (rl & 15);
        }
        w = (second ? p.w1 : p.w0) + (size_t)rr * (size_t)(p.k >> 1);
        sc = (second ? p.s1 : p.s0) + (size_t)rr * (size_t)p.scols;
    };
    {   // records of this K range -> LDS by direct loads (a wave instruction
        // moves one KiB: lane l's 16 bytes land at lrec + 1024 c + 16 l)
        const uint8_t *src = p.rec + (size_t)b0 * BS;
        const int bytes = nb * BS;   // a multiple of 16
        for (int c = wave; c * 1024 < bytes; c += NW)
            if (c * 1024 + lane * 16 < bytes)
                __builtin_amdgcn_global_load_lds(src + c * 1024 + lane * 16, lrec + c * 1024, 16,
                                                 0, 0);
    }
    const uint8_t *wr[R];
    const float *sr[R];
    int rows[R];
#pragma unroll
    for (int rb = 0; rb < R; ++rb) {
        const int rl = wave * 16 * R + 16 * rb + i;
        rows[rb] = blockIdx.x * ROWS + rl;
        row_ptrs(rl, wr[rb], sr[rb]);
    }
    f32x4 acc[R];
#pragma unroll
    for (int rb = 0; rb < R; ++rb) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Weights of one batch: lane (i, q) takes the 16 bytes of group q of its
    // row (cached, not non-temporal: each load takes half of a row's 128-byte
    // line and the next batch takes the other half).
    auto load_w = [&](int k0, u32x4 (&wv)[R]) {
#pragma unroll
        for (int rb = 0; rb < R; ++rb)
            wv[rb] = *reinterpret_cast<const u32x4 *>(wr[rb] + (k0 >> 1) + 16 * q);
    };
    // Scales of a quad of 4 batches from k0: lane (i, q) takes the 4 group
    // scales of batch q of its row -- one 16-byte load when SV (group 32, one
    // 64-byte piece of a row per 4 lanes), else one load per group.  (A dword
    // per lane per batch made every 128-byte scale line eight 16-byte
    // requests; the streams of scales then cost almost as much as the weights.)
    auto load_s = [&](int k0, f32x4 (&sv)[R]) {
        const int kb = min(k0 + q * kBatch, klast);
#pragma unroll
        for (int rb = 0; rb < R; ++rb) {
            if (SV) {
                sv[rb] = *reinterpret_cast<const f32x4 *>(sr[rb] + (kb >> 5));
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) sv[rb][t] = sr[rb][(kb + 32 * t) >> p.gshift];
            }
        }
    };

    // The f32 path of a flagged batch: (q - 8) x in IEEE arithmetic on the raw
    // activations (v_mfma_f32_16x16x4_f32: lane l supplies A[l % 16][l / 16]
    // and B[l / 16][l % 16]).
    auto compute_f32 = [&](int k0, const u32x4 (&wv)[R], const f32x4 (&st)[R]) {
        const int xr = T == 1 ? (i < 8 ? i : kLimbMaxM) : i;
        const float *xrow = p.x + (size_t)(xr < p.m ? xr : 0) * p.k;
        const bool live = xr < p.m;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float *xp = xrow + k0 + 32 * t + 8 * q;
            const float4 a = *reinterpret_cast<const float4 *>(xp);
            const float4 b = *reinterpret_cast<const float4 *>(xp + 4);
            const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int rb = 0; rb < R; ++rb) {
                f32x4 D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    D = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        live ? xv[e] : 0.f, (float)((wv[rb][t] >> (4 * e)) & 15u) - 8.0f, D, 0,
                        0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[rb][r] = fmaf(D[r], st[rb][t], acc[rb][r]);
            }
        }
    };
    const h8 boff = offset_operand();
    // The four steps of a batch are independent until the accumulation: all
    // LDS reads first, then the four offset MFMAs, then per row block the four
    // weight MFMAs; the batch's partial sum takes the batch exponent once.
    auto compute = [&](int k0, const u32x4 (&wv)[R], const f32x4 (&st)[R]) {
        const uint8_t *rg = lrec + (size_t)((k0 - ks) / kBatch) * BS;
        // exponent bytes of A-rows 4 q .. 4 q + 3, both halves
        const uint2 pw = *reinterpret_cast<const uint2 *>(rg + 4 * T * kTile + 8 * q);
        float pf[2][4];   // 2^(24 - e) of the lane's four A-rows, per half
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                pf[h][r] = __builtin_bit_cast(
                    float, __builtin_amdgcn_ubfe(r < 2 ? pw.x : pw.y, 16 * (r & 1) + 8 * h, 8)
                               << 23);
        // one half batch (groups 2 h, 2 h + 1) at a time: half the A tiles and
        // offsets live at once
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            h8 A[2][T];
#pragma unroll
            for (int g = 0; g < 2; ++g)
#pragma unroll
                for (int u = 0; u < T; ++u)
                    A[g][u] =
                        *reinterpret_cast<const h8 *>(rg + ((2 * h + g) * T + u) * kTile + lane * 16);
            f32x4 off[2][T];
#pragma unroll
            for (int g = 0; g < 2; ++g)
#pragma unroll
                for (int u = 0; u < T; ++u)
                    off[g][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        A[g][u], boff, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int rb = 0; rb < R; ++rb) {
                f32x4 D[2];
#pragma unroll
                for (int g = 0; g < 2; ++g) {
                    const h8 B = expand_nibbles(wv[rb][2 * h + g]);
                    D[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[g][0], B, off[g][0], 0, 0, 0);
                    if (T == 2)
                        D[g] += __builtin_amdgcn_mfma_f32_16x16x32_f16(A[g][T - 1], B,
                                                                       off[g][T - 1], 0, 0, 0);
                }
                f32x4 bs = D[0] * st[rb][2 * h];
#pragma unroll
                for (int r = 0; r < 4; ++r) bs[r] = fmaf(D[1][r], st[rb][2 * h + 1], bs[r]);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[rb][r] = fmaf(bs[r], pf[h][r], acc[rb][r]);
            }
        }
    };
    // Batch jj of a quad: transpose its weights, gather the row's four scales
    // from lane (i, jj) (ds_bpermute), then the f16 MFMA or, for a flagged
    // batch (only when CHECK), the f32 path.
    auto step = [&](auto check, int k0, u32x4 (&wv)[R], const f32x4 (&sv)[R], int jj) {
        f32x4 st[R];
#pragma unroll
        for (int rb = 0; rb < R; ++rb) {
            transpose4(wv[rb]);
#pragma unroll
            for (int t = 0; t < 4; ++t) st[rb][t] = __shfl(sv[rb][t], i + 16 * jj);
        }
        if (decltype(check)::value && flagged(lrec + (size_t)((k0 - ks) / kBatch) * BS + 4 * T * kTile))
            compute_f32(k0, wv, st);
        else
            compute(k0, wv, st);
    };

    // Quads of 4 batches, DQ - 1 quads ahead in a register ring, issued with
    // the record copy so the block pays one memory latency before its first
    // batch; the records come from LDS, so each later wait is for the oldest
    // weights only.  Loads past the range re-read its last batch: every pass
    // of the main loop issues the same loads, which keeps the compiler's waits
    // exact, and it runs whole quads only, so its batches are straight-line
    // code the compiler can interleave (no per-batch branch).
    const int nq = (nb + 3) / 4, nqf = nb / 4;
    u32x4 wq[DQ][4][R];
    f32x4 sq[DQ][R];
    auto load_quad = [&](int qd, u32x4 (&wv)[4][R], f32x4 (&sv)[R]) {
        const int kq = ks + 4 * min(qd, nq - 1) * kBatch;
#pragma unroll
        for (int j = 0; j < 4; ++j) load_w(min(kq + j * kBatch, klast), wv[j]);
        load_s(kq, sv);
    };
    // The record copy above must be issued before the kAfter weight and scale
    // loads the wait below counts: the empty asm keeps the compiler from
    // moving any of them across (none of them can be merged: their addresses
    // are 64 bytes apart or runtime-strided).
    asm volatile("" ::: "memory");
#pragma unroll
    for (int j = 0; j < DQ - 1; ++j) load_quad(j, wq[j], sq[j]);
    // Wait for this wave's record copy only: vector loads retire in order, so
    // the kAfter weight and scale loads issued after it may stay in flight.
    constexpr int kAfter = (DQ - 1) * (4 * R + (SV ? R : 4 * R));
    static_assert(kAfter < 64, "vmcnt holds 6 bits");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((kAfter & 15) | ((kAfter >> 4) << 14) | (7 << 4) | (15 << 8));
    asm volatile("" ::: "memory");
    __syncthreads();   // every wave's copy landed
    // NaN / Inf flags of the range, once, from the records in LDS (a batch for
    // the f32 path has exponent byte 0; nb <= 64): the common all-finite case
    // needs no per-batch test.
    const bool any_bad =
        __any(lane < nb && flagged(lrec + (size_t)(lane < nb ? lane : 0) * BS + 4 * T * kTile)) != 0;
    auto run = [&](auto check) {
        int qd = 0;
        for (; qd + DQ <= nqf; qd += DQ) {
#pragma unroll
            for (int j = 0; j < DQ; ++j) {
                load_quad(qd + j + DQ - 1, wq[(j + DQ - 1) % DQ], sq[(j + DQ - 1) % DQ]);
#pragma unroll
                for (int jj = 0; jj < 4; ++jj)
                    step(check, ks + (4 * (qd + j) + jj) * kBatch, wq[j][jj], sq[j], jj);
            }
        }
        // the last quads (the last may be partial): slot j holds quad qd + j
        if (qd + DQ - 1 < nq) load_quad(qd + DQ - 1, wq[DQ - 1], sq[DQ - 1]);
#pragma unroll
        for (int j = 0; j < DQ; ++j)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const int k0 = ks + (4 * (qd + j) + jj) * kBatch;
                if (k0 < ke) step(check, k0, wq[j][jj], sq[j], jj);
            }
    };
    if (any_bad) run(std::true_type{});
    else run(std::false_type{});

    // Lane l's register r holds A-row 4 (l / 16) + r of weight row l % 16; for
    // T = 1 rows 8..15 are the second limbs of rows 0..7 (lanes l + 32).
    if constexpr (PE) {
        // gate and up values to LDS past the records ([8 tokens][64 columns]
        // each, then h in rows padded to 65), one h per thread, then the
        // record's half by four waves, one group and four slots each
        float *gb = reinterpret_cast<float *>(lrec + (size_t)nb * BS);
        float *ub = gb + 8 * kPairCols, *hb = ub + 8 * kPairCols;
        f32x4 v = acc[0];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] += __shfl_down(v[r], 32);
        if (lane < 32) {   // tokens 4 q + r of column 16 (wave / 2) + i
            float *dst = (wave & 1) ? ub : gb;
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[(4 * q + r) * kPairCols + 16 * (wave >> 1) + i] = v[r];
        }
        const int col = kPairCols * blockIdx.x + lane, tok = wave;
        const float bg = p.b0 ? p.b0[col] : 0.f, bu = p.b1 ? p.b1[col] : 0.f;
        __syncthreads();
        const float h = silu(gb[tok * kPairCols + lane] + bg) * (ub[tok * kPairCols + lane] + bu);
        if (tok < p.m) p.y[(size_t)tok * p.n + col] = h;
        hb[tok * (kPairCols + 1) + lane] = h;
        if (!p.rec_out) return;
        __syncthreads();
        if (wave >= 4) return;
        const int tr = i & 7;
        float hv[2][8];
        float mx = 0.f;
        bool fin = true;
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                hv[g][e] = tr < p.m ? hb[tr * (kPairCols + 1) + 32 * g + 8 * q + e] : 0.f;
                fin = fin && __builtin_isfinite(hv[g][e]);
                mx = fmaxf(mx, fabsf(hv[g][e]));
            }
        const HalfExp he = half_exp(mx, fin);
        const int half = blockIdx.x & 1, g = wave >> 1;
        uint8_t *rg = p.rec_out + (size_t)(blockIdx.x >> 1) * BS;
        auto part = [&](auto s0) {   // slots s0 .. s0 + 3 of group g
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            h4 l1, l2;
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const int j = decltype(s0)::value + jj;
                const float x = g ? hv[1][slot_elem(j)] : hv[0][slot_elem(j)];
                _Float16 a, b;
                limbs_of(x, he, j, a, b);
                l1[jj] = a;
                l2[jj] = b;
            }
            *reinterpret_cast<h4 *>(rg + (size_t)(2 * half + g) * kTile + lane * 16 +
                                    2 * decltype(s0)::value) = i < 8 ? l1 : l2;
        };
        if (wave & 1) part(std::integral_constant<int, 4>{});
        else part(std::integral_constant<int, 0>{});
        if (wave == 0 && q == 0) rg[4 * kTile + 2 * i + half] = he.byte;
        return;
    }
    float *pp = part + (size_t)split * (size_t)p.m * (size_t)ntot;
#pragma unroll
    for (int rb = 0; rb < R; ++rb) {
        f32x4 v = acc[rb];
        if (T == 1) {
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] += __shfl_down(v[r], 32);
        }
        if (rows[rb] < ntot && (T == 2 || q < 2)) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tok = 4 * q + r;
                if (tok < p.m) pp[(size_t)tok * ntot + rows[rb]] = v[r];
            }
        }
    }
}

// y = sum of the split partials (split order) + bias (+ residual).  res may
// be y (an in-place residual add): each element is read before it is written,
// by the same thread, so neither pointer is restrict-qualified.
__global__ __launch_bounds__(256) void k_limb_reduce(const float *__restrict__ part, int splits,
                                                     int m, int n, const float *__restrict__ b0,
                                                     const float *res, float *y) {
    const size_t total = (size_t)m * n;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (size_t)gridDim.x * blockDim.x) {
        const int row = (int)(e % (size_t)n);
        const float bias = b0 ? b0[row] : 0.f, r0 = res ? res[e] : 0.f;
        // eight splits' loads in flight at a time, summed in split order
        float g = 0.f;
        int s = 0;
        for (; s + 8 <= splits; s += 8) {
            float t[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) t[j] = part[(size_t)(s + j) * total + e];
#pragma unroll
            for (int j = 0; j < 8; ++j) g += t[j];
        }
        for (; s < splits; ++s) g += part[(size_t)s * total + e];
        if (b0) g += bias;
        if (res) g += r0;
        y[e] = g;
    }
}

// SwiGLU pair: h = silu(gate + b0) * (up + b1) from the split partials of the
// stacked [gate; up] rows.  One block per 128-row batch of h: each thread sums
// 4 T contiguous values of one token over the splits (four splits' loads in
// flight at a time) and writes them to y and LDS; waves 0 and 1 then write
// the two halves of the batch's record for the next projection (rec_out,
// K = n).
template <int T>
__global__ __launch_bounds__(256) void k_limb_reduce_pair(const float *__restrict__ part,
                                                          int splits, int m, int n,
                                                          const float *__restrict__ b0,
                                                          const float *__restrict__ b1,
                                                          float *__restrict__ y,
                                                          uint8_t *__restrict__ rec_out) {
    constexpr int TOKS = 8 * T;           // tokens of the batch
    constexpr int PER = 32 / T;           // threads per token
    // rows padded by one float: the record wave reads the 8 (16) tokens of a
    // column in one instruction, which would otherwise hit one bank
    __shared__ float hs[TOKS][kBatch + 1];
    const int tid = threadIdx.x, bt = blockIdx.x;
    const int tok = tid / PER, c0 = (tid % PER) * 4 * T;   // 4 T values at rows c0..
    const int row0 = kBatch * bt + c0;
    const size_t ntot = 2 * (size_t)n;
    const size_t plane = (size_t)m * ntot;
    const bool live = tok < m;
    f32x4 gs[T] = {}, us[T] = {};
    if (live) {
        const float *pg = part + (size_t)tok * ntot + row0;
        int s = 0;
        for (; s + 4 <= splits; s += 4) {
            f32x4 lg[4][T], lu[4][T];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int h = 0; h < T; ++h) {
                    lg[j][h] = *reinterpret_cast<const f32x4 *>(pg + (s + j) * plane + 4 * h);
                    lu[j][h] = *reinterpret_cast<const f32x4 *>(pg + (s + j) * plane + n + 4 * h);
                }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int h = 0; h < T; ++h) {
                    gs[h] += lg[j][h];
                    us[h] += lu[j][h];
                }
        }
        for (; s < splits; ++s)
#pragma unroll
            for (int h = 0; h < T; ++h) {
                gs[h] += *reinterpret_cast<const f32x4 *>(pg + s * plane + 4 * h);
                us[h] += *reinterpret_cast<const f32x4 *>(pg + s * plane + n + 4 * h);
            }
        // biases before any store: on this GPU loads and stores retire through
        // one in-order counter, so a load issued after a store waits for it
        f32x4 bg[T] = {}, bu[T] = {};
#pragma unroll
        for (int h = 0; h < T; ++h) {
            if (b0) bg[h] = *reinterpret_cast<const f32x4 *>(b0 + row0 + 4 * h);
            if (b1) bu[h] = *reinterpret_cast<const f32x4 *>(b1 + row0 + 4 * h);
        }
#pragma unroll
        for (int h = 0; h < T; ++h) {
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = silu(gs[h][e] + bg[h][e]) * (us[h][e] + bu[h][e]);
            *reinterpret_cast<f32x4 *>(y + (size_t)tok * n + row0 + 4 * h) = v;
#pragma unroll
            for (int e = 0; e < 4; ++e) hs[tok][c0 + 4 * h + e] = v[e];
        }
    }
    if (!rec_out) return;
    __syncthreads();
    if (tid >= 128) return;
    // waves 0 and 1: halves 0 and 1 of the batch's record
    const int lane = tid & 63, h = tid >> 6, i = lane & 15, q = lane >> 4;
    const int tr = T == 1 ? (i & 7) : i;
    float v[2][8];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) v[g][e] = tr < m ? hs[tr][32 * (2 * h + g) + 8 * q + e] : 0.f;
    build_half<T>(v, lane, rec_out + (size_t)bt * rec_stride(T), h);
}

constexpr int kTargetBlocks = 512;

struct Plan {
    int ksl, splits, r, chunks, nw;
    bool pe;   // a pair whose kernel writes h and its records (no reduce)
    size_t lds;
};

// Whole-K form: when the records of the whole K fit kLdsWhole and there are
// enough row blocks, one block per CU (kWholeWaves waves, one 16-row block each)
// runs the whole K with no split: every record byte is copied to LDS once per
// CU and there are no split partials to add.  A SwiGLU pair takes eight waves,
// the gate and up rows of 64 columns of h, and runs the epilogue itself (one
// more wave per block than a single projection, about 1 us on the Llama-3-8B
// gate/up at M = 8, against the 4.7 us of the reduce kernel it removes).
constexpr int kWholeWaves = 7;
// Ring depth in quads: one quad in flight while the previous one computes.
// (Two or three quads ahead measured slower in every form, 17.7 -> 19.1 ->
// 20.4 us for the Llama-3-8B gate/up pair at M = 8.)
constexpr int kQuads = 2;
constexpr int kLdsWhole = 132 << 10;

// Otherwise four waves per block, each over R 16-row blocks (R = 2 when the
// grid would otherwise exceed about kTargetBlocks blocks); the K split is as
// long as the block's records fit kLdsBudget.
Plan plan(int m, int n, int k, bool pair) {
    Plan pl;
    const int bs = rec_stride(tiles_of(m));
    const int batches = k / kBatch;
    const long ntot = pair ? 2L * n : n;
    if (tiles_of(m) == 1 && (long)batches * bs <= kLdsWhole &&
        ntot / 16 >= (long)kWholeWaves * kTargetBlocks * 3 / 8) {
        pl.pe = pair;
        pl.nw = pair ? kPairWaves : kWholeWaves;
        pl.r = 1;
        pl.splits = 1;
        pl.ksl = k;
        // a pair's epilogue: gate, up and a padded h tile past the records
        pl.lds = (size_t)batches * bs +
                 (pair ? (size_t)(8 * (3 * kPairCols + 1)) * sizeof(float) : 0);
        pl.chunks = pair ? n / kPairCols
                         : (int)((ntot + 16 * kWholeWaves - 1) / (16 * kWholeWaves));
        return pl;
    }
    pl.pe = false;
    pl.nw = 4;
    int per = kLdsBudget / bs;
    if (per < 1) per = 1;
    if (per > batches) per = batches;
    pl.splits = (batches + per - 1) / per;
    per = (batches + pl.splits - 1) / pl.splits;   // even out the splits
    pl.splits = (batches + per - 1) / per;
    pl.ksl = per * kBatch;
    pl.lds = (size_t)per * bs;
    const long want_rows = (ntot * pl.splits + kTargetBlocks - 1) / kTargetBlocks;
    pl.r = want_rows > 96 ? 2 : 1;
    const int rows = 16 * pl.r * pl.nw;
    pl.chunks = (int)((ntot + rows - 1) / rows);
    return pl;
}

template <int T>
__global__ __launch_bounds__(256) void k_limb_prep(const float *__restrict__ x,
                                                   uint8_t *__restrict__ rec, int m, int k,
                                                   int batches) {
    limb_prep_body<T>(x, rec, m, k, batches);
}


// ---------------------------------------------------------------------------
// Batched projection for M >= 17 on the same exact limbs: the tiling of the
// FP32-MFMA kernel (w4_mfma.hip) with its f32 operands replaced.  A block (4
// waves) owns 64 weight rows (16 per wave) x MT 16-row slabs of activation
// rows x a K range (split-K; the partials go to k_mfma_reduce in the FP32
// kernel's layout, so the epilogues are shared).  Per 128-element batch:
//   * the MT slab records of the batch (limb_prep's two-tile format, built
//     per 16-row slab by lgemm_prep) are staged in LDS through registers,
//     loaded one batch ahead, and read by all four waves;
//   * each lane loads one 16-byte chunk of its weight row (group q of the
//     batch) and its scale; a 4x4 transpose across the lane quarters leaves
//     dword q of group t in register t, expanded to the f16 B operand;
//   * per slab and group: two offset MFMAs (the -8 of every weight, against
//     the limbs) and two weight MFMAs (one per limb), each exact; the group's
//     result takes the row's group scale, and each half batch its 2^(24 - e);
//   * a slab whose half batch is flagged (NaN / Inf, or out of range) takes
//     the f32 path on the raw activations for that batch.
// The f16 matrix cores run 16x the FP32 rate, and two limbs plus the offset
// MFMAs cost 4 instructions per group and slab against 8 of
// v_mfma_f32_16x16x4_f32 at a quarter of the K each.
template <int MT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void k_w4_lgemm(LGemmArgs a) {
    constexpr int BS = rec_stride(2);             // 8224 bytes per slab and batch
    constexpr int ACH = 4 * 2 * kTile / 16;       // 16-byte chunks of a slab's A tiles (512)
    constexpr int AV = MT * ACH / 256;            // A chunks per thread per batch
    static_assert(MT * ACH % 256 == 0, "whole chunks per thread");
    __shared__ __align__(16) uint8_t lr[MT * BS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int i = lane & 15, q = lane >> 4;
    int bx = blockIdx.x;
    const int second = bx >= a.nbx ? 1 : 0;   // dual launch: blocks of the up projection
    bx -= second * a.nbx;
    const uint8_t *w = second ? a.w1 : a.w0;
    const float *s = second ? a.s1 : a.s0;
    const int sb = blockIdx.z * MT;                   // first slab of the block
    const int ms = min(MT, a.nslabs - sb);            // slabs that exist
    const int kb = blockIdx.y * a.klen;
    const int ke = min(a.k, kb + a.klen);
    const int row = bx * 64 + wave * 16 + i;
    const bool rok = row < a.n;
    const uint8_t *wrow = w + (size_t)(rok ? row : 0) * (size_t)(a.k >> 1);
    const float *srow = s + (size_t)(rok ? row : 0) * (size_t)a.scols;
    const size_t slab_bytes = (size_t)a.batches * BS;

    u32x4 ar[AV];   // the next batch's record chunks
    u32x4 tr;       // its exponent tail chunk (threads < 2 MT)
    u32x4 wr;
    float sr;
    auto load_step = [&](int k0) {
        const int bt = k0 / kBatch;
#pragma unroll
        for (int v = 0; v < AV; ++v) {
            const int f = tid + 256 * v, mt = f / ACH, c = f - mt * ACH;
            ar[v] = mt < ms ? *reinterpret_cast<const u32x4 *>(a.rec + (size_t)(sb + mt) * slab_bytes +
                                                               (size_t)bt * BS + 16 * c)
                            : u32x4{0u, 0u, 0u, 0u};
        }
        {
            const int mt = tid >> 1;
            tr = (tid < 2 * MT && mt < ms)
                     ? *reinterpret_cast<const u32x4 *>(a.rec + (size_t)(sb + mt) * slab_bytes +
                                                        (size_t)bt * BS + 8 * kTile + 16 * (tid & 1))
                     : u32x4{0u, 0u, 0u, 0u};
        }
        const int kk = k0 + 32 * q;
        wr = rok ? load_nt16(wrow + (kk >> 1)) : u32x4{0u, 0u, 0u, 0u};
        sr = rok ? srow[kk >> a.gshift] : 0.f;
    };

    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const h8 boff = offset_operand();

    load_step(kb);
    for (int k0 = kb; k0 < ke; k0 += kBatch) {
        __syncthreads();   // the previous batch's readers are done with lr
#pragma unroll
        for (int v = 0; v < AV; ++v) {
            const int f = tid + 256 * v, mt = f / ACH, c = f - mt * ACH;
            *reinterpret_cast<u32x4 *>(lr + mt * BS + 16 * c) = ar[v];
        }
        if (tid < 2 * MT) *reinterpret_cast<u32x4 *>(lr + (tid >> 1) * BS + 8 * kTile + 16 * (tid & 1)) = tr;
        u32x4 cw = wr;
        const float sc = sr;
        __syncthreads();
        if (k0 + kBatch < ke) load_step(k0 + kBatch);
        transpose4(cw);
        float st[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) st[t] = __shfl(sc, i + 16 * t);
        h8 B[4];
        B[0] = expand_nibbles(cw.x);
        B[1] = expand_nibbles(cw.y);
        B[2] = expand_nibbles(cw.z);
        B[3] = expand_nibbles(cw.w);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            if (mt >= ms) break;
            const uint8_t *rg = lr + mt * BS;
            if (flagged(rg + 8 * kTile)) {
                // f32 path: tokens of the slab's rows, raw activations
                const int tok = (sb + mt) * 16 + i;
                const bool live = tok < a.m;
                const float *xrow = a.x + (size_t)(live ? tok : 0) * a.k;
                const uint32_t dw[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const float *xp = xrow + k0 + 32 * t + 8 * q;
                    const float4 a0 = *reinterpret_cast<const float4 *>(xp);
                    const float4 a1 = *reinterpret_cast<const float4 *>(xp + 4);
                    const float xv[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                    f32x4 D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        D = __builtin_amdgcn_mfma_f32_16x16x4f32(
                            live ? xv[e] : 0.f, (float)((dw[t] >> (4 * e)) & 15u) - 8.0f, D, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[mt][r] = fmaf(D[r], st[t], acc[mt][r]);
                }
                continue;
            }
            const uint2 pw = *reinterpret_cast<const uint2 *>(rg + 8 * kTile + 8 * q);
            // one half batch (groups 2 h, 2 h + 1) at a time
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                h8 A[2][2];
#pragma unroll
                for (int g = 0; g < 2; ++g)
#pragma unroll
                    for (int u = 0; u < 2; ++u)
                        A[g][u] = *reinterpret_cast<const h8 *>(rg + ((2 * h + g) * 2 + u) * kTile +
                                                                lane * 16);
                f32x4 D[2];
#pragma unroll
                for (int g = 0; g < 2; ++g) {
                    const f32x4 o0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        A[g][0], boff, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    const f32x4 o1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        A[g][1], boff, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    D[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[g][0], B[2 * h + g], o0, 0, 0, 0);
                    D[g] += __builtin_amdgcn_mfma_f32_16x16x32_f16(A[g][1], B[2 * h + g], o1, 0, 0, 0);
                }
                f32x4 bs = D[0] * st[2 * h];
#pragma unroll
                for (int r = 0; r < 4; ++r) bs[r] = fmaf(D[1][r], st[2 * h + 1], bs[r]);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float pf = __builtin_bit_cast(
                        float, __builtin_amdgcn_ubfe(r < 2 ? pw.x : pw.y, 16 * (r & 1) + 8 * h, 8) << 23);
                    acc[mt][r] = fmaf(bs[r], pf, acc[mt][r]);
                }
            }
        }
    }

    const int col = bx * 64 + wave * 16 + i;
    if (col >= a.n) return;
    float *pb = a.part + (size_t)(second * a.splits + blockIdx.y) * (size_t)a.m * a.n;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int mr = (sb + mt) * 16 + 4 * q + r;
            if (mr < a.m) pb[(size_t)mr * a.n + col] = acc[mt][r];
        }
    }
}

// Records of x [m, k] as 16-row slabs in the two-tile format: slab s at
// rec + s * (k / 128) * rec_stride(2).
__global__ __launch_bounds__(256) void k_lgemm_prep(const float *__restrict__ x,
                                                    uint8_t *__restrict__ rec, int m, int k,
                                                    int batches) {
    const int sl = blockIdx.y;
    limb_prep_body<2>(x + (size_t)sl * 16 * k, rec + (size_t)sl * batches * rec_stride(2),
                      min(16, m - 16 * sl), k, batches);
}

}  // namespace

size_t lgemm_records_bytes(int m, int k) {
    return (size_t)((m + 15) / 16) * (size_t)(k / kBatch) * (size_t)rec_stride(2);
}

int lgemm_prep(const float *x, uint8_t *rec, int m, int k, hipStream_t st) {
    TB_REQUIRE(m >= 1 && k % kBatch == 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: slab records need K % 128 == 0");
    const int batches = k / kBatch;
    const dim3 grid((unsigned)((2 * batches + 3) / 4), (unsigned)((m + 15) / 16));
    hipLaunchKernelGGL(k_lgemm_prep, grid, dim3(256), 0, st, x, rec, m, k, batches);
    TB_LAUNCHED();
    return TB_OK;
}

int lgemm_launch(const LGemmArgs &a, int mt, dim3 grid, hipStream_t st) {
    switch (mt) {
        case 1: hipLaunchKernelGGL(k_w4_lgemm<1>, grid, dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL(k_w4_lgemm<2>, grid, dim3(256), 0, st, a); break;
        case 3: hipLaunchKernelGGL(k_w4_lgemm<3>, grid, dim3(256), 0, st, a); break;
        default: hipLaunchKernelGGL(k_w4_lgemm<4>, grid, dim3(256), 0, st, a); break;
    }
    TB_LAUNCHED();
    return TB_OK;
}

size_t limb_records_bytes(int m, int k) {
    return (size_t)(k / kBatch) * (size_t)rec_stride(tiles_of(m));
}

size_t limb_partials_bytes(int m, int n, int k, bool pair) {
    const Plan pl = plan(m, n, k, pair);
    if (pl.pe) return 0;
    return (size_t)pl.splits * (size_t)m * (size_t)(pair ? 2 * n : n) * sizeof(float);
}

bool limb_shape_ok(int64_t m, int64_t n, int64_t k, bool pair) {
    if (m < 1 || m > kLimbMaxM || n < 1 || k < kBatch || k % kBatch != 0) return false;
    if (k > (int64_t)1 << 24 || n > (int64_t)1 << 23) return false;
    return !pair || n % kBatch == 0;   // the pair reduce takes whole 128-row batches of h
}

int limb_prep(const float *x, uint8_t *rec, int m, int k, hipStream_t st) {
    TB_REQUIRE(m >= 1 && m <= kLimbMaxM && k % kBatch == 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: activation records need 1 <= M <= 16 and K % 128 == 0");
    const int batches = k / kBatch;
    const dim3 grid((unsigned)((2 * batches + 3) / 4));   // one wave per half batch
    if (tiles_of(m) == 1)
        hipLaunchKernelGGL(k_limb_prep<1>, grid, dim3(256), 0, st, x, rec, m, k, batches);
    else
        hipLaunchKernelGGL(k_limb_prep<2>, grid, dim3(256), 0, st, x, rec, m, k, batches);
    TB_LAUNCHED();
    return TB_OK;
}

int w4_limb(const LimbParams &p, float *part, hipStream_t st) {
    const bool pair = p.w1 != nullptr;
    TB_REQUIRE(limb_shape_ok(p.m, p.n, p.k, pair), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: small-batch MFMA projection needs 1 <= M <= 16, K % 128 == 0 "
               "(and N % 128 == 0 for a SwiGLU pair)");
    const bool t1 = tiles_of(p.m) == 1;
    const int ntot = pair ? 2 * p.n : p.n;
    const Plan pl = plan(p.m, p.n, p.k, pair);
    // group-32 scales in 16-byte rows: one vector load per lane per quad
    const bool sv = p.gshift == 5 && p.scols == (p.k >> 5) &&
                    (reinterpret_cast<uintptr_t>(p.s0) & 15) == 0 &&
                    (!pair || (reinterpret_cast<uintptr_t>(p.s1) & 15) == 0);
    // more than the default 64 KiB of dynamic LDS for the whole-K forms (set
    // per call: the attribute belongs to the current device's code object)
#define TB_LIMB_LDS(T_, R_, NW_, D_, SV_, PE_)                                                  \
    TB_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_w4_limb<T_, R_, NW_, D_, SV_, PE_>), \
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)pl.lds))
#define TB_LIMB_GO(T_, R_, NW_, D_, PE_)                                                        \
    do {                                                                                        \
        const dim3 g_((unsigned)pl.chunks, (unsigned)pl.splits), b_(64 * NW_);                  \
        if (sv) {                                                                               \
            if (pl.lds > kLdsBudget) TB_LIMB_LDS(T_, R_, NW_, D_, true, PE_);                   \
            hipLaunchKernelGGL((k_w4_limb<T_, R_, NW_, D_, true, PE_>), g_, b_, pl.lds, st, p,  \
                               part, pl.ksl, ntot);                                             \
        } else {                                                                                \
            if (pl.lds > kLdsBudget) TB_LIMB_LDS(T_, R_, NW_, D_, false, PE_);                  \
            hipLaunchKernelGGL((k_w4_limb<T_, R_, NW_, D_, false, PE_>), g_, b_, pl.lds, st, p, \
                               part, pl.ksl, ntot);                                             \
        }                                                                                       \
    } while (0)
    if (pl.pe) {
        TB_LIMB_GO(1, 1, kPairWaves, kQuads, true);
    } else if (pl.nw == kWholeWaves) {
        TB_LIMB_GO(1, 1, kWholeWaves, kQuads, false);
    } else if (pl.r == 2) {
        if (t1) TB_LIMB_GO(1, 2, 4, kQuads, false);
        else TB_LIMB_GO(2, 2, 4, kQuads, false);
    } else {
        if (t1) TB_LIMB_GO(1, 1, 4, kQuads, false);
        else TB_LIMB_GO(2, 1, 4, kQuads, false);
    }
#undef TB_LIMB_GO
#undef TB_LIMB_LDS
    TB_LAUNCHED();
    if (pl.pe) return TB_OK;
    if (pair) {
        const dim3 rg((unsigned)(p.n / kBatch));
        if (t1)
            hipLaunchKernelGGL(k_limb_reduce_pair<1>, rg, dim3(256), 0, st, part, pl.splits, p.m,
                               p.n, p.b0, p.b1, p.y, p.rec_out);
        else
            hipLaunchKernelGGL(k_limb_reduce_pair<2>, rg, dim3(256), 0, st, part, pl.splits, p.m,
                               p.n, p.b0, p.b1, p.y, p.rec_out);
    } else {
        const size_t total = (size_t)p.m * (size_t)p.n;
        const unsigned nb = (unsigned)std::min<size_t>((total + 255) / 256, 2048);
        hipLaunchKernelGGL(k_limb_reduce, dim3(nb), dim3(256), 0, st, part, pl.splits, p.m, p.n,
                           p.b0, p.res, p.y);
    }
    TB_LAUNCHED();
    return TB_OK;
}

}  // namespace tb

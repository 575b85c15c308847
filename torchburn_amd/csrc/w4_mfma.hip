// Batched grouped-INT4 projection Y[M, N] = X[M, K] . deq(W)^T on FP32 MFMA
// (v_mfma_f32_16x16x4_f32), for batches of M >= 5 rows (16-row tiles), where
// the work is a dense contraction.
//
// Replaces the M > 1 path of the reference's w4a32_grouped_linear
// (src/quantization/packed_v2.rs:557-624 -> gemm_w4a32_grouped,
// src/quantization/gemv.rs:1690-1725), which runs one full GEMV per activation
// row and so reads the weights M times; here every weight byte is read once per
// 64 activation rows.  The batched SwiGLU of fused_swiglu_mlp_batched_w4a32
// (src/quantization/fused_ops.rs:1267-1319: gate GEMM, up GEMM, silu * up,
// down GEMM) maps onto the dual launch plus the SwiGLU reduce epilogue.
//
// Tiling.  A block (4 waves) owns 64 weight rows (16 per wave) x up to 64
// activation rows (MT tiles of 16) x a K range of `klen` (split-K over blocks,
// partial sums reduced by k_mfma_reduce in a fixed order, so results are
// deterministic).  Per 128-wide K step:
//   * X [16*MT, 128] is staged once per block in LDS (row pitch 132 floats,
//     so the 16 rows of an MFMA operand read fall on distinct banks) and read
//     by all four waves;
//   * each lane loads one 16-byte chunk of its weight row (32 nibbles = one
//     group at g32, half of one at g64) plus the group scale, and dequantizes
//     it in registers straight into the MFMA B operand: (nib - 8) * s as
//     fma(nib, s, -8 s).  Each weight element is used by exactly one wave, so
//     staging W in LDS would only add traffic.
//   * MFMA operand layout (16x16x4, one block): lane l supplies A[l % 16][l / 16]
//     and B[l / 16][l % 16]; D[4 (l / 16) + r][l % 16] comes back in register r.
//     The four lane groups q = l / 16 take K sub-ranges 32q..32q+31 of the step,
//     so one MFMA consumes element e of each group's 32; the K order inside a
//     contraction is free as long as A and B agree.
//   * the next step's X tile, weight chunk and scale are loaded into registers
//     before the current step's MFMAs are issued; X tiles alternate between two
//     LDS buffers, so each step needs one barrier;
//   * up to four independent accumulators per 16-row tile keep dependent MFMAs
//     apart (small M has few tiles to interleave).
//   * V2: weights in the v2 stream (34-byte group-64 blocks with f16 scales,
//     packed_v2.rs:26-143): a lane's 16-byte chunk is one half of a block,
//     read with dword-aligned loads and a funnel shift (load_v2_chunk).
#include <float.h>
#include <stdlib.h>

#include "gemv_common.hpp"
#include "tb_common.hpp"
#include "w4_gemv.hpp"
#include "w4_limb.hpp"
#include "w4_mfma.hpp"

namespace tb {

using namespace gemv;

namespace {

constexpr int kBN = 64;        // weight rows per block
constexpr int kBK = 128;       // K per step
constexpr int kXP = kBK + 4;   // LDS row pitch of the X tile (floats)
constexpr int kTargetBlocks = 512;   // split-K target (TB_MFMA_BLOCKS overrides, tuning only)

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int MT, bool V2>
__global__ __launch_bounds__(256) void k_w4_mfma(const float *__restrict__ x,
                                                 const uint8_t *__restrict__ w0,
                                                 const float *__restrict__ s0,
                                                 const uint8_t *__restrict__ w1,
                                                 const float *__restrict__ s1,
                                                 float *__restrict__ part, int m, int n, int k,
                                                 int scols, int gshift, int klen, int nbx,
                                                 int splits) {
    constexpr int XV = MT * 2;             // float4 of the X tile per thread
    constexpr int NACC = MT <= 2 ? 4 : 2;  // independent accumulation chains per M tile
    constexpr int NB = MT <= 2 ? 2 : 1;    // X tile buffers (two cost occupancy at MT >= 3)
    __shared__ float xs[NB][MT * 16 * kXP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int bx = blockIdx.x;
    const int second = bx >= nbx ? 1 : 0;   // dual launch: blocks of the up projection
    bx -= second * nbx;
    const uint8_t *w = second ? w1 : w0;
    const float *s = second ? s1 : s0;
    const int m0 = blockIdx.z * MT * 16;
    const int kb = blockIdx.y * klen;
    const int ke = min(k, kb + klen);
    const int row = bx * kBN + wave * 16 + (lane & 15);
    const int q = lane >> 4;
    const bool rok = row < n;
    const uint8_t *wrow = w + (size_t)(rok ? row : 0) * (size_t)(k >> 1);
    // scales of the row at srow[kk >> gshift]: scols per row (k / group, or 1 per
    // row / 0 for one scalar with gshift 31)
    const float *srow = V2 ? nullptr : s + (size_t)(rok ? row : 0) * (size_t)scols;
    const uint32_t vrow = (uint32_t)(rok ? row : 0) * (uint32_t)((k >> 6) * kV2Block);

    float4 xr[XV];
    u32x4 wr;
    float sr;
    auto load_step = [&](int k0) {
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            const int f = tid + 256 * i;
            const int r = f >> 5, c = (f & 31) * 4;
            const bool ok = (m0 + r < m) && (k0 + c < ke);
            xr[i] = ok ? *reinterpret_cast<const float4 *>(x + (size_t)(m0 + r) * k + k0 + c)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        const int kk = k0 + 32 * q;
        const bool ok = rok && kk < ke;
        if (V2) {
            const int kc = ok ? kk : 0;   // addresses stay inside the stream
            const uint32_t blk = vrow + (uint32_t)(kc >> 6) * kV2Block;
            wr = ok ? load_v2_chunk(w, blk + (uint32_t)((kc >> 5) & 1) * 16u)
                    : u32x4{0u, 0u, 0u, 0u};
            sr = ok ? load_v2_scale(w, blk) : 0.f;
        } else {
            wr = ok ? load_nt16(wrow + (kk >> 1)) : u32x4{0u, 0u, 0u, 0u};
            sr = ok ? srow[kk >> gshift] : 0.f;
        }
    };

    f32x4 acc[MT][NACC];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int c = 0; c < NACC; ++c) acc[t][c] = f32x4{0.f, 0.f, 0.f, 0.f};

    load_step(kb);
    int buf = 0;
    for (int k0 = kb; k0 < ke; k0 += kBK, buf ^= (NB - 1)) {
        float *xb = xs[buf];
        // With two buffers, `buf` was last read two steps ago, before the
        // previous step's barrier; with one, wait for this step's readers.
        if (NB == 1) __syncthreads();
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            const int f = tid + 256 * i;
            *reinterpret_cast<float4 *>(xb + (f >> 5) * kXP + (f & 31) * 4) = xr[i];
        }
        const u32x4 cw = wr;
        const float sc = sr;
        __syncthreads();
        if (k0 + kBK < ke) load_step(k0 + kBK);
        const float nsc = -8.0f * sc;
        const uint32_t dws[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            float a[MT][8];
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const float *xa = xb + (t * 16 + (lane & 15)) * kXP + 32 * q + 8 * d;
                const float4 a0 = *reinterpret_cast<const float4 *>(xa);
                const float4 a1 = *reinterpret_cast<const float4 *>(xa + 4);
                a[t][0] = a0.x; a[t][1] = a0.y; a[t][2] = a0.z; a[t][3] = a0.w;
                a[t][4] = a1.x; a[t][5] = a1.y; a[t][6] = a1.z; a[t][7] = a1.w;
            }
            const uint32_t lo = dws[d] & 0x0F0F0F0Fu, hi = (dws[d] >> 4) & 0x0F0F0F0Fu;
            float b[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                b[2 * i] = fmaf((float)((lo >> (8 * i)) & 0xFFu), sc, nsc);
                b[2 * i + 1] = fmaf((float)((hi >> (8 * i)) & 0xFFu), sc, nsc);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e)
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    acc[t][e % NACC] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        a[t][e], b[e], acc[t][e % NACC], 0, 0, 0);
        }
    }

    const int col = bx * kBN + wave * 16 + (lane & 15);
    if (col >= n) return;
    float *pb = part + (size_t)(second * splits + blockIdx.y) * (size_t)m * n;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        f32x4 v = acc[t][0];
#pragma unroll
        for (int c = 1; c < NACC; ++c) v += acc[t][c];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int mr = m0 + t * 16 + 4 * q + r;
            if (mr < m) pb[(size_t)mr * n + col] = v[r];
        }
    }
}

// Sum of the split-K partials in split order, then the epilogue.  res may be
// y (an in-place residual add; each element is read before the same thread
// writes it), so neither pointer is restrict-qualified.
__global__ __launch_bounds__(256) void k_mfma_reduce(const float *__restrict__ part, int splits,
                                                     int m, int n, const float *__restrict__ b0,
                                                     const float *__restrict__ b1,
                                                     const float *res, float *y, int epi) {
    const size_t total = (size_t)m * n;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int col = (int)(i % (size_t)n);
        float g = 0.f;
        for (int s = 0; s < splits; ++s) g += part[(size_t)s * total + i];
        if (b0) g += b0[col];
        if (epi == EPI_SWIGLU) {
            float u = 0.f;
            for (int s = 0; s < splits; ++s) u += part[(size_t)(splits + s) * total + i];
            if (b1) u += b1[col];
            y[i] = silu(g) * u;
        } else {
            if (epi == EPI_RESID) g += res[i];
            y[i] = g;
        }
    }
}

struct Plan {
    int mt, mz, nbx, klen, splits;
};

int target_blocks() {
    static int v = [] {
        const char *e = getenv("TB_MFMA_BLOCKS");
        const int t = e ? atoi(e) : 0;
        return t > 0 ? t : kTargetBlocks;
    }();
    return v;
}

Plan plan(int m, int n, int k, bool dual) {
    Plan pl;
    const int tiles = (m + 15) / 16;
    pl.mt = tiles < 4 ? tiles : 4;
    pl.mz = (tiles + pl.mt - 1) / pl.mt;
    pl.nbx = (n + kBN - 1) / kBN;
    const int blocks = pl.nbx * (dual ? 2 : 1) * pl.mz;
    const int steps = (k + kBK - 1) / kBK;
    int want = (target_blocks() + blocks - 1) / blocks;
    if (want > steps) want = steps;
    if (want < 1) want = 1;
    const int per = (steps + want - 1) / want;
    pl.klen = per * kBK;
    pl.splits = (k + pl.klen - 1) / pl.klen;
    return pl;
}

// From 17 rows the projection runs on the exact f16 limbs of x (k_w4_lgemm,
// w4_limb.hip) when K is whole 128-element batches and a 32-element group has
// one scale (16-row projections measured 14.7 against 14.4 us on FP32 MFMA);
// TB_MFMA_LIMB=0 keeps the FP32-MFMA kernel (measurement only).
bool use_limbs(int m, int k, bool v2, int scale_mode, int gshift) {
    static const bool on = [] {
        const char *e = getenv("TB_MFMA_LIMB");
        return !(e && e[0] == '0');
    }();
    return on && m >= 17 && !v2 && k % kBK == 0 && (scale_mode != 0 || gshift >= 5);
}

size_t partials_only(int m, int n, int k, bool dual) {
    const Plan pl = plan(m, n, k, dual);
    return (size_t)(dual ? 2 : 1) * pl.splits * (size_t)m * n * sizeof(float);
}

}  // namespace

size_t w4_mfma_partials_bytes(int m, int n, int k, bool dual) {
    // partials, then (256-byte aligned) room for the limb records of x
    const size_t pb = (partials_only(m, n, k, dual) + 255) & ~(size_t)255;
    return pb + (m >= 17 && k % kBK == 0 ? lgemm_records_bytes(m, k) : 0);
}

int w4_mfma(const MfmaParams &p, int epi, float *part, hipStream_t st) {
    const bool dual = p.w1 != nullptr;
    TB_REQUIRE(p.k % 32 == 0 && p.m >= 1 && p.n >= 1, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: MFMA projection needs K % 32 == 0");
    if (p.v2)
        TB_REQUIRE(p.k % 64 == 0 && ((uintptr_t)p.w0 & 3u) == 0 &&
                       (!dual || ((uintptr_t)p.w1 & 3u) == 0) &&
                       (size_t)p.n * (size_t)(p.k / 64) * kV2Block < (1ull << 32),
                   TB_ERR_UNSUPPORTED,
                   "TB_UNSUPPORTED: v2 blocks need K % 64 == 0, a 4-byte aligned stream "
                   "under 4 GiB");
    const Plan pl = plan(p.m, p.n, p.k, dual);
    dim3 grid(pl.nbx * (dual ? 2 : 1), pl.splits, pl.mz);
    const int scols = p.scale_mode == 0 ? p.k >> p.gshift : (p.scale_mode == 1 ? 1 : 0);
    const int gsh = p.scale_mode == 0 ? p.gshift : 31;
    if (use_limbs(p.m, p.k, p.v2, p.scale_mode, p.gshift)) {
        LGemmArgs a;
        a.x = p.x;
        a.rec = reinterpret_cast<uint8_t *>(part) +
                ((partials_only(p.m, p.n, p.k, dual) + 255) & ~(size_t)255);
        a.w0 = p.w0; a.s0 = p.s0; a.w1 = p.w1; a.s1 = p.s1;
        a.part = part;
        a.m = p.m; a.n = p.n; a.k = p.k;
        a.scols = scols; a.gshift = gsh;
        a.klen = pl.klen; a.nbx = pl.nbx; a.splits = pl.splits;
        a.batches = p.k / kBK;
        a.nslabs = (p.m + 15) / 16;
        int rc = lgemm_prep(p.x, const_cast<uint8_t *>(a.rec), p.m, p.k, st);
        if (rc) return rc;
        if ((rc = lgemm_launch(a, pl.mt, grid, st))) return rc;
    } else {
#define TB_MFMA_LAUNCH(MT)                                                                   \
    if (p.v2)                                                                                \
        hipLaunchKernelGGL((k_w4_mfma<MT, true>), grid, dim3(256), 0, st, p.x, p.w0, p.s0,   \
                           p.w1, p.s1, part, p.m, p.n, p.k, scols, gsh, pl.klen, pl.nbx,     \
                           pl.splits);                                                       \
    else                                                                                     \
        hipLaunchKernelGGL((k_w4_mfma<MT, false>), grid, dim3(256), 0, st, p.x, p.w0, p.s0,  \
                           p.w1, p.s1, part, p.m, p.n, p.k, scols, gsh, pl.klen, pl.nbx,     \
                           pl.splits)
    switch (pl.mt) {
        case 1: TB_MFMA_LAUNCH(1); break;
        case 2: TB_MFMA_LAUNCH(2); break;
        case 3: TB_MFMA_LAUNCH(3); break;
        default: TB_MFMA_LAUNCH(4); break;
    }
#undef TB_MFMA_LAUNCH
    TB_LAUNCHED();
    }
    const size_t total = (size_t)p.m * p.n;
    size_t blocks = (total + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(k_mfma_reduce, dim3((unsigned)blocks), dim3(256), 0, st, part, pl.splits,
                       p.m, p.n, p.b0, dual ? p.b1 : nullptr, p.res, p.y,
                       dual ? (int)EPI_SWIGLU : epi);
    TB_LAUNCHED();
    return TB_OK;
}

}  // namespace tb

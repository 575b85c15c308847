// Grouped INT4 (W4A32) GEMV for gfx950: one pass takes 1 or 2 activation rows.
//
// Replaces gemv_w4a32_grouped / gemm_w4a32_grouped (reference
// src/quantization/gemv.rs:1514-1725), the SwiGLU neuron kernels
// (src/quantization/gemv/swiglu.rs:205-289, driven by
// src/quantization/fused_ops.rs:244-407) and the residual add that follows the
// O and down projections (src/llm/decoder.rs:1235-1238, 1344-1347).
//
// Work mapping (one wavefront = 64 lanes):
//   * A row of K elements is cut into 32-element chunks (16 bytes of nibbles,
//     exactly one group-32 group).  Lane `cl` of wave `ks` owns chunk
//     ks*SW + cl for the whole block, so its slice of x is loaded once.
//   * The K-slices of one row are spread over the waves of the block (split-K
//     across wavefronts).  Rows with fewer than 64 chunks share a wave: `rps`
//     rows side by side, one per lane span of 2^b.
//   * Each row step a lane issues one coalesced non-temporal 128-bit load of
//     packed nibbles (consecutive lanes read consecutive 16-byte pieces of the
//     same row: a wave instruction covers 1 KiB of one row) and one f32 scale.
//   * x arrives as chunk records (k_xquant / fused producers): a 23-bit
//     fixed-point integer per element as six signed base-16 digit planes
//     (two's complement nibbles, [-8, 7]).  With no
//     records given (XR: one activation row, one matrix), each lane builds
//     its chunk's record itself from the raw x it loads, while its weight
//     loads are in flight, which saves the separate record pass.  The stored
//     nibble q becomes the signed nibble q - 8 with one XOR by 8 per nibble,
//     and then
//        sum_i (q_i - 8) X_i = sum_l 16^l * v_dot8_i32_i4(q ^ 0x8..8, digit_l)
//     directly on the packed nibbles -- no unpacking, no correction terms --
//     exact in 32-bit integers; each 16-element half is rounded to f32 once,
//     scaled by its step, and the chunk partial by its group scale.
//   * The per-lane partials of J rows are transpose-reduced across lanes,
//     summed across waves through LDS, and the epilogue (bias, residual add, or
//     silu(g)*u of a gate/up pair) writes the outputs.
//   * A wave whose x chunk holds NaN/Inf takes an f32 path instead (the
//     reference's unpack-and-fma), so non-finite values propagate.
//   * V2: the weights are the v2 stream (34-byte group-64 blocks with f16
//     scales, packed_v2.rs:26-143; gemv_w4a32_grouped_v2, packed_v2.rs:326-485).
//     A chunk is one half of a block: its 16 nibble bytes come from five
//     dword-aligned loads and a funnel shift, its scale from the block's two
//     trailing bytes; the arithmetic is unchanged.
#include "gemv_common.hpp"
#include "tb_common.hpp"

namespace tb {

using namespace gemv;

namespace {

template <int M, int J, bool DUAL, int EPI, bool V2, bool XR>
struct W4Gemv {
    static constexpr int D = DUAL ? 2 : 1;
    static constexpr int V = D * J * M;
    static constexpr int NDW = 4;   // dwords of nibbles per 32-element chunk

    // One batch of J rows (x D matrices): raw nibble chunks, raw scales and a
    // bit per row, clear for idle lanes and rows past N (their scale becomes 0
    // when the batch is consumed, not when issued, so issuing never waits).
    struct Batch {
        uint32_t q[D][J][NDW];
        float sc[D][J];
        uint32_t ok;
    };

    // The lane's x chunk records (one per activation row), or with XR its
    // 32 raw activations.
    struct XRec {
        u32x4 limbs[M][6];
        u32x4 tail[M];   // {step 0-15, step 16-31, sum 0-15, sum 16-31}
        float4 raw[XR ? M : 1][8];
    };

    const W4Params &p;
    const Layout &L;
    int lane, wave, grp, rr, cl, chunk;
    bool act;
    size_t bpr, boff, soff;
    int gcols, sg;
    uint32_t limb[M][6][NDW];   // limb[m][l][d] nibble e = digit l of X_{8d+e}
    float sx[M][2];             // power-of-two step of each half
    bool finite;                // false -> the wave takes the f32 path

    __device__ __forceinline__ W4Gemv(const W4Params &pp, const Layout &ll) : p(pp), L(ll) {
        lane = threadIdx.x & 63;
        wave = threadIdx.x >> 6;
        grp = wave / L.nks;
        rr = lane >> L.b;
        cl = lane & ((1 << L.b) - 1);
        const int chunk_raw = (wave - grp * L.nks) * L.sw + cl;
        act = (cl < L.sw) && (chunk_raw < L.c);
        // Idle lanes read a valid chunk and contribute zero (scale forced to 0).
        chunk = act ? chunk_raw : 0;
        // scale of (row, chunk) at s[row * gcols + sg]: per group, per row or one
        gcols = p.scale_mode == 0 ? p.k >> p.gshift : (p.scale_mode == 1 ? 1 : 0);
        sg = p.scale_mode == 0 ? (chunk * 32) >> p.gshift : 0;
        if (V2) {
            bpr = (size_t)(p.k >> 6) * kV2Block;
            soff = (size_t)(chunk >> 1) * kV2Block;   // the chunk's block
            boff = soff + (size_t)(chunk & 1) * 16;
        } else {
            bpr = (size_t)(p.k >> 1);
            soff = 0;
            boff = (size_t)chunk * 16;
        }
    }

    __device__ __forceinline__ void issue_x(XRec &xr) const {
        if (XR) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const int mm = m < p.m ? m : 0;
                const float4 *xp =
                    reinterpret_cast<const float4 *>(p.x + (size_t)mm * p.k + chunk * 32);
#pragma unroll
                for (int i = 0; i < 8; ++i) xr.raw[m][i] = xp[i];
            }
            return;
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const int mm = m < p.m ? m : 0;
            // quad i of this chunk's record: row base + (i * c + chunk) * 4 dwords
            const u32x4 *rp = reinterpret_cast<const u32x4 *>(p.xq + (size_t)mm * L.c * kXRecDwords) +
                              chunk;
#pragma unroll
            for (int i = 0; i < 6; ++i) xr.limbs[m][i] = rp[(size_t)i * L.c];
            xr.tail[m] = rp[(size_t)6 * L.c];
        }
    }

    __device__ __forceinline__ void unpack_x(const XRec &xr) {
        bool fin = true;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            if (XR) {
                float v[32];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    v[4 * i] = xr.raw[m][i].x; v[4 * i + 1] = xr.raw[m][i].y;
                    v[4 * i + 2] = xr.raw[m][i].z; v[4 * i + 3] = xr.raw[m][i].w;
                }
                lane_chunk_rec(v, limb[m], sx[m]);
                fin = fin && (m >= p.m || !(__builtin_isnan(sx[m][0]) || __builtin_isnan(sx[m][1])));
                continue;
            }
#pragma unroll
            for (int l = 0; l < 6; ++l) {
                const u32x4 t = xr.limbs[m][l];
                limb[m][l][0] = t.x; limb[m][l][1] = t.y; limb[m][l][2] = t.z; limb[m][l][3] = t.w;
            }
            sx[m][0] = __uint_as_float(xr.tail[m].x);
            sx[m][1] = __uint_as_float(xr.tail[m].y);
            fin = fin && (m >= p.m || !(__builtin_isnan(sx[m][0]) || __builtin_isnan(sx[m][1])));
        }
        // One vote per wave, so the integer path runs without per-lane branches.
        finite = __all(fin ? 1 : 0) != 0;
    }

    // f32 chunk dot for a wave whose x holds NaN/Inf: sum (n - 8) * x_i as the
    // reference's unpack-and-fma does.
    __device__ __forceinline__ float chunk_dot_f32(const uint32_t (&q)[NDW], int m) const {
        const float4 *xp = reinterpret_cast<const float4 *>(p.x + (size_t)m * p.k + chunk * 32);
        float acc = 0.f;
#pragma unroll
        for (int dw = 0; dw < NDW; ++dw) {
            const float4 a = xp[2 * dw], b = xp[2 * dw + 1];
            const float xe[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                acc = fmaf((float)((int)((q[dw] >> (4 * e)) & 15u) - 8), xe[e], acc);
        }
        return acc;
    }

    // Issues every load of batch `blk` (J*D 16-byte chunks + scales per lane).
    __device__ __forceinline__ void issue(int blk, Batch &bt) const {
        const int row0 = blk * L.rpb;
        bt.ok = 0u;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int row_raw = row0 + grp * L.jr + j * L.rps + rr;
            const bool ok = act && row_raw < p.n;
            bt.ok |= ok ? (1u << j) : 0u;
            // rows past N re-read row 0 with weight 0
            const int row = !ok ? 0 : (EPI == EPI_ROPE ? rope_row(row_raw, p.rope.hd) : row_raw);
            // 32-bit offsets from the uniform bases (weights < 4 GiB, checked
            // at launch): one VGPR per address, SGPR-based addressing.
            const uint32_t wo = (uint32_t)row * (uint32_t)bpr + (uint32_t)boff;
            const uint32_t so = ((uint32_t)row * (uint32_t)gcols + (uint32_t)sg) * 4u;
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const uint8_t *wb = d ? p.w1 : p.w0;
                u32x4 v;
                if (V2) {
                    v = load_v2_chunk(wb, wo);
                    bt.sc[d][j] = load_v2_scale(wb, (uint32_t)row * (uint32_t)bpr + (uint32_t)soff);
                } else {
                    v = load_nt16(wb + wo);
                    bt.sc[d][j] = *reinterpret_cast<const float *>(
                        reinterpret_cast<const char *>(d ? p.s1 : p.s0) + so);
                }
                bt.q[d][j][0] = v.x; bt.q[d][j][1] = v.y; bt.q[d][j][2] = v.z; bt.q[d][j][3] = v.w;
            }
        }
    }

    // Dot products of the batch, per 16-element half h of the chunk:
    //   sum_i (n_i - 8) X_i = sum_l 16^l a_l,  a_l = signed dot8 of (n - 8, digit l)
    // exact in 32-bit integers (|a_l| <= 1024, every Horner partial below 2^31,
    // the sum below 2^29); one f32 rounding per half, then * step, summed,
    // * group scale.
    __device__ __forceinline__ void dots(const Batch &bt, float (&v)[V]) const {
        if (!finite) {
#pragma unroll
            for (int j = 0; j < J; ++j)
#pragma unroll
                for (int d = 0; d < D; ++d)
#pragma unroll
                    for (int m = 0; m < M; ++m)
                        v[(d * J + j) * M + m] =
                            ((bt.ok >> j) & 1u) && m < p.m
                                ? bt.sc[d][j] * chunk_dot_f32(bt.q[d][j], m)
                                : 0.f;
            return;
        }
        // Rows in load order, JG at a time: the dots of the first rows start
        // as soon as their weights are in (loads retire in issue order).
        // Within a group, Horner from the top digit with every (row, matrix,
        // activation row, half) chain side by side: the shifted running sum is
        // the accumulator of the next dot8 (the accumulate-in-place v_dot8c
        // needs no zeroed register), and with at least 4 chains consecutive
        // dot8s never depend on each other, so the dot-to-dot accumulator
        // hazard costs no wait states.
        constexpr int JG = (D * M * 2 >= 4 || J < 2) ? 1 : 2;
#pragma unroll
        for (int j0 = 0; j0 < J; j0 += JG) {
            int qs[JG][D][NDW];   // signed nibbles n - 8
#pragma unroll
            for (int jj = 0; jj < JG; ++jj)
#pragma unroll
                for (int d = 0; d < D; ++d)
#pragma unroll
                    for (int dw = 0; dw < NDW; ++dw)
                        qs[jj][d][dw] = (int)(bt.q[d][j0 + jj][dw] ^ 0x88888888u);
            int t[JG][D][M][2];
#pragma unroll
            for (int l = 5; l >= 0; --l) {
#pragma unroll
                for (int hw = 0; hw < 2; ++hw)   // dword 2h + hw of each half
#pragma unroll
                    for (int jj = 0; jj < JG; ++jj)
#pragma unroll
                        for (int d = 0; d < D; ++d)
#pragma unroll
                            for (int m = 0; m < M; ++m)
#pragma unroll
                                for (int h = 0; h < 2; ++h) {
                                    int &a = t[jj][d][m][h];
                                    const int acc = l == 5 ? (hw ? a : 0)
                                                           : (hw ? a : (int)((uint32_t)a << 4));
                                    a = __builtin_amdgcn_sdot8(qs[jj][d][2 * h + hw],
                                                               (int)limb[m][l][2 * h + hw], acc,
                                                               false);
                                }
            }
#pragma unroll
            for (int jj = 0; jj < JG; ++jj)
#pragma unroll
                for (int d = 0; d < D; ++d)
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const int j = j0 + jj;
                        const float sc = ((bt.ok >> j) & 1u) ? bt.sc[d][j] : 0.f;
                        v[(d * J + j) * M + m] =
                            sc * fmaf(sx[m][0], (float)t[jj][d][m][0],
                                      sx[m][1] * (float)t[jj][d][m][1]);
                    }
        }
    }
};

// One block = one batch of J rows.  Order matters: x record loads, then the
// batch's weight and scale loads, then the epilogue operands, then the dot
// products (which wait only for what they read, since loads retire in issue
// order).  Straight-line code: a
// loop back-edge would make the compiler drain the load counter early.
template <int M, int J, bool DUAL, int EPI, bool V2, bool XR, int NW>
__global__ __launch_bounds__(NW * 64) void k_w4_gemv(W4Params p, Layout L, Epi e) {
    using G = W4Gemv<M, J, DUAL, EPI, V2, XR>;
    __shared__ float red[NW * 64];
    __shared__ EpiShared sh;
    G g(p, L);
    typename G::Batch a;
    typename G::XRec xr;
    const int row0 = blockIdx.x * L.rpb;
    const int pos = epi_pos<EPI>(e);
    g.issue_x(xr);
    __builtin_amdgcn_sched_barrier(0);
    g.issue(blockIdx.x, a);
    __builtin_amdgcn_sched_barrier(0);
    const EpiIn in = epi_load<J, M, DUAL, EPI>(L, row0, e, pos);
    __builtin_amdgcn_sched_barrier(0);
    g.unpack_x(xr);
    float v[G::V];
    g.dots(a, v);
    reduce_and_store<G::V, J, M, DUAL, EPI>(v, red, sh, L, g.lane, g.wave, row0, e, in);
}

// Chunk records of x [m, k]: eight lanes per (row, 32-element chunk).
__global__ __launch_bounds__(256) void k_xquant(const float *__restrict__ x,
                                               uint32_t *__restrict__ xq, int m, int k) {
    const int c = k / 32;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int rec = t >> 3, sub = t & 7;
    const bool live = rec < m * c;   // whole 8-lane groups are live or not
    const int row = live ? rec / c : 0, ch = live ? rec - row * c : 0;
    const float4 v = live ? reinterpret_cast<const float4 *>(x + (size_t)row * k + ch * 32)[sub]
                          : make_float4(0.f, 0.f, 0.f, 0.f);
    build_xrec8(v, sub, live, xq + (size_t)row * c * kXRecDwords, c, ch);
}

// NW: the block's wave limit (kMaxWaves, or kMaxWavesWide for more row
// groups per block in kernels within 128 VGPRs).
template <int M, int J, bool DUAL, int EPI, bool V2 = false, bool XR = false, int NW = kMaxWaves>
int launch(const W4Params &p, hipStream_t st) {
    constexpr int V = (DUAL ? 2 : 1) * J * M;
    static_assert(V <= 64, "at most 64 partials per lane");
    Layout L;
    const bool prod = p.rec_out || p.xw_out || p.ssq_out;
    TB_REQUIRE(make_layout(p.k / 32, Log2<V>::value, J, L, prod ? 16 : 0, NW), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: w4a32 GEMV supports K <= " + std::to_string(kMaxWaves * 64 * 32));
    Epi e{};
    e.b0 = p.b0; e.b1 = p.b1; e.res = p.res; e.y = p.y; e.n = p.n; e.m = p.m; e.rope = p.rope;
    e.ssq_in = p.ssq_in; e.ssq_n = p.ssq_n; e.eps = p.eps;
    e.inv_h = p.norm_h > 0 ? 1.0f / (float)p.norm_h : 0.f;
    e.rec_out = p.rec_out; e.rec_w = p.rec_w; e.xw_out = p.xw_out; e.ssq_out = p.ssq_out;
    // n floats of any valid buffer: the scales (n * k / group), or the v2 stream
    e.any = V2 ? reinterpret_cast<const float *>(p.w0) : p.s0;
    if (p.ssq_in)
        TB_REQUIRE(p.m == 1 && p.ssq_n <= kMaxSsqPerThread * L.nwaves * 64, TB_ERR_UNSUPPORTED,
                   "TB_UNSUPPORTED: fused RMSNorm input needs M == 1 and K == H");
    if (prod)
        TB_REQUIRE(p.m == 1 && EPI != EPI_ROPE && L.rpb % 16 == 0 && L.rpb <= kMaxRecRows &&
                       p.n % 32 == 0,
                   TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: records of the output need M == 1, "
                                       "N % 32 == 0 and 16-row blocks");
    if (EPI == EPI_ROPE)
        TB_REQUIRE(p.m == 1 && p.rope.hd % L.rpb == 0 && L.rpb % 2 == 0 && p.n % p.rope.hd == 0,
                   TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: fused RoPE needs whole rotation pairs per block");
    const size_t wbytes = V2 ? (size_t)(p.k / 64) * kV2Block : (size_t)(p.k / 2);
    TB_REQUIRE((size_t)p.n * wbytes < (1ull << 32), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: w4 GEMV weights must be under 4 GiB");
    if (V2)
        TB_REQUIRE(p.k % 64 == 0 && !DUAL && ((uintptr_t)p.w0 & 3u) == 0, TB_ERR_UNSUPPORTED,
                   "TB_UNSUPPORTED: v2 blocks need K % 64 == 0 and a 4-byte aligned stream");
    const int grid = (p.n + L.rpb - 1) / L.rpb;
    if (XR)
        TB_REQUIRE(p.x && ((uintptr_t)p.x & 15u) == 0 && p.ssq_in == nullptr, TB_ERR_UNSUPPORTED,
                   "TB_UNSUPPORTED: w4 GEMV without x records needs a 16-byte aligned x "
                   "and no fused RMSNorm input");
    hipLaunchKernelGGL((k_w4_gemv<M, J, DUAL, EPI, V2, XR, NW>), dim3(grid), dim3(L.nwaves * 64),
                       0, st, p, L, e);
    TB_LAUNCHED();
    return TB_OK;
}

// Blocks of a single-matrix M = 1 launch at j rows per block.
int blocks_at(const W4Params &p, int j) {
    Layout L;
    if (!make_layout(p.k / 32, ceil_log2(j), j, L, 0)) return 0;
    return (p.n + L.rpb - 1) / L.rpb;
}

template <bool DUAL, int EPI, bool V2 = false>
int dispatch_m(const W4Params &p, hipStream_t st) {
    // x stays in VGPRs, so one pass takes <= 4 rows.  Rows per block at M = 1:
    // 8 for a gate/up pair (with the dots in load order, 8 rows measured
    // 15.4 us against 16.0 at 4 and 16.7 at 16 for Llama-3-8B); 16 for one
    // matrix whose epilogue writes records (16-row pieces); otherwise the
    // largest of 16, 8, 4 that still gives 512 blocks (two per CU: the
    // Qwen2.5-0.5B up-projection [4864, 896] 5.9 -> 4.7 us at 4 rows, the
    // Llama-3-8B down projection 10.0 -> 9.0 us at 8).
    if (p.m <= 1) {
        const bool prod = p.rec_out || p.xw_out || p.ssq_out;
        // A single matrix whose epilogue writes records needs 16-row blocks;
        // with 3 or more K-slice waves, row groups of 8 or 4 rows in
        // 1024-thread blocks give it two to four times the waves of 16 rows
        // in one group (Llama-3-8B down: 7 K-slices x 2 groups of 8 rows).
        const int nks = (p.k / 32 + 63) / 64;
        if (!DUAL && !V2 && prod && !p.rows_j && p.xq && EPI != EPI_ROPE && nks >= 3) {
            if (nks > 4) return launch<1, 8, false, EPI, false, false, kMaxWavesWide>(p, st);
            return launch<1, 4, false, EPI, false, false, kMaxWavesWide>(p, st);
        }
        int j = p.rows_j;
        if (!j) {
            j = DUAL ? 8 : 16;
            if (!DUAL && !prod)
                while (j > 4 && blocks_at(p, j) < 512) j /= 2;
            // With one or two K-slice waves, 4 rows per row group (groups of
            // 4 rows x the K slices, two groups to the 16-row block): the
            // Qwen2.5-0.5B O projection [896, 896] takes 56 two-wave blocks
            // instead of 28 one-wave ones, decode 1094 -> 1121 tok/s; the
            // Llama-3-8B O projection measured the same either way.
            if (!DUAL && prod && nks <= 2) j = 4;
        }
        if (!DUAL && !p.xq) {   // records built in the kernel from x
            if (j == 4) return launch<1, 4, false, EPI, V2, true>(p, st);
            if (j == 16) return launch<1, 16, false, EPI, V2, true>(p, st);
            return launch<1, 8, false, EPI, V2, true>(p, st);
        }
        if (j == 4) return launch<1, 4, DUAL, EPI, V2>(p, st);
        if (j == 16) return launch<1, 16, DUAL, EPI, V2>(p, st);
        return launch<1, 8, DUAL, EPI, V2>(p, st);
    }
    // 2 and 3-4 activation rows: fewer weight rows per block as the records
    // (28 VGPRs per activation row) and the dot products grow with M.
    if (p.m <= 2) return launch<2, DUAL ? 4 : 8, DUAL, EPI, V2>(p, st);
    return launch<4, DUAL ? 2 : 4, DUAL, EPI, V2>(p, st);
}

}  // namespace

int xquant(const float *x, uint32_t *xq, int m, int k, hipStream_t st) {
    const int n = m * (k / 32) * 8;   // 8 lanes per chunk record
    if (n == 0) return TB_OK;
    hipLaunchKernelGGL(k_xquant, dim3((n + 255) / 256), dim3(256), 0, st, x, xq, m, k);
    TB_LAUNCHED();
    return TB_OK;
}

int w4_gemv(W4Params p, int epi, hipStream_t st) {
    TB_REQUIRE(p.m >= 1 && p.m <= kMaxW4RowsPerPass, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: w4 GEMV pass takes 1..4 rows");
    TB_REQUIRE(p.k % 32 == 0, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: w4 GEMV needs K % 32 == 0");
    TB_REQUIRE(p.xq || (p.m == 1 && epi != EPI_ROPE && p.w1 == nullptr), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: w4 GEMV: x records are required for M > 1, gate/up pairs and "
               "fused RoPE");
    if (p.v2) {
        TB_REQUIRE(p.w1 == nullptr, TB_ERR_UNSUPPORTED,
                   "TB_UNSUPPORTED: v2 blocks take single projections");
        if (epi == EPI_RESID) return dispatch_m<false, EPI_RESID, true>(p, st);
        if (epi == EPI_ROPE) {
            if (p.rows_j == 8) return launch<1, 8, false, EPI_ROPE, true>(p, st);
            if (p.rows_j == 16) return launch<1, 16, false, EPI_ROPE, true>(p, st);
            return launch<1, 4, false, EPI_ROPE, true>(p, st);
        }
        return dispatch_m<false, EPI_PLAIN, true>(p, st);
    }
    if (p.w1 != nullptr) return dispatch_m<true, EPI_SWIGLU>(p, st);
    if (epi == EPI_RESID) return dispatch_m<false, EPI_RESID>(p, st);
    if (epi == EPI_ROPE) {
        // QKV: 4 rows per block (the K/Q/V projection is small, so more and
        // shorter waves; Llama-3-8B decode 2.10-2.13 -> 2.06 ms per token
        // against 16 rows).
        if (p.rows_j == 8) return launch<1, 8, false, EPI_ROPE>(p, st);
        if (p.rows_j == 16) return launch<1, 16, false, EPI_ROPE>(p, st);
        return launch<1, 4, false, EPI_ROPE>(p, st);
    }
    return dispatch_m<false, EPI_PLAIN>(p, st);
}

}  // namespace tb

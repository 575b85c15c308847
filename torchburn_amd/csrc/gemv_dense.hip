// INT8 per-channel (W8A32) and FP32 GEMV for gfx950, 1 or 2 activation rows
// per pass.
//
// Replaces gemv_w8a32 / w8a32_linear (reference src/quantization/gemv.rs:733-1061,
// row dot dot_f32_i8 at gemv.rs:280-324), the INT8 SwiGLU neuron loop of
// fused_swiglu_mlp_w8a32 (src/quantization/fused_ops.rs:8-133), and the fp32
// lm_head of the per-layer Python path (python/torchburn/llm/model.py:499-500).
//
// Same work mapping as the INT4 kernel (w4_gemv.hip): 32 elements per lane for
// the life of the block, split-K over waves, J rows per block, a transpose
// reduction and one epilogue.  Differences:
//   * a lane's 32 elements are LD 16-byte pieces strided by the lanes of its
//     row (piece cl + sw * i of its wave's K slice), so each load instruction
//     reads one contiguous run of the row; 32 contiguous elements per lane
//     would spread one instruction over 64 cache lines (fp32 lm_head: 2.2
//     TB/s);
//   * x stays in VGPRs as f32 (32 per activation row), loaded from x directly;
//   * INT8: two non-temporal 16-byte loads per chunk; each signed byte becomes
//     a float in one instruction (v_cvt_f32_i32 with a sign-extending byte
//     select), so the row dot is summed over w * x itself, without an offset
//     to cancel; the per-channel scale multiplies the row dot in the epilogue
//     (y = dot * s + b, as gemv.rs:777-785);
//   * FP32: eight 16-byte loads per chunk, one FMA per element.
#include "gemv_common.hpp"
#include "gemv_dense.hpp"
#include "tb_common.hpp"

namespace tb {

using namespace gemv;

namespace {

template <int WT, int M, int J, bool DUAL, int EPI>
struct DenseGemv {
    static constexpr int D = DUAL ? 2 : 1;
    static constexpr int V = D * J * M;
    static constexpr int LD = WT == W_I8 ? 2 : 8;   // 16-byte loads per chunk
    static constexpr int BPE = WT == W_I8 ? 1 : 4;  // bytes per weight element

    struct Batch {
        u32x4 q[D][J][LD];
        uint32_t ok;
    };

    static constexpr int PE = 16 / BPE;             // elements per 16-byte piece

    const DenseParams &p;
    const Layout &L;
    int lane, wave, grp, rr, cl;
    bool act;
    size_t bpr;
    int piece[LD];        // the lane's pieces (clamped into the row)
    uint32_t pmask;       // bit i: piece i lies inside K
    float xr[M][32];

    __device__ __forceinline__ DenseGemv(const DenseParams &pp, const Layout &ll) : p(pp), L(ll) {
        lane = threadIdx.x & 63;
        wave = threadIdx.x >> 6;
        grp = wave / L.nks;
        rr = lane >> L.b;
        cl = lane & ((1 << L.b) - 1);
        const int pbase = (wave - grp * L.nks) * L.sw * LD;   // first piece of the K slice
        const int npieces = L.c * LD;
        pmask = 0u;
#pragma unroll
        for (int i = 0; i < LD; ++i) {
            const int pc = pbase + cl + L.sw * i;
            const bool in = cl < L.sw && pc < npieces;
            pmask |= in ? (1u << i) : 0u;
            piece[i] = in ? pc : npieces - 1;
        }
        act = pmask != 0u;
        bpr = (size_t)p.k * BPE;
    }

    // x pieces of the lane (PE floats each); pieces past K read as zero.
    __device__ __forceinline__ void issue_x(float4 (&raw)[M][8]) const {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float *xm = p.x + (size_t)(m < p.m ? m : 0) * p.k;
#pragma unroll
            for (int i = 0; i < LD; ++i) {
                const float4 *xp = reinterpret_cast<const float4 *>(xm + (size_t)piece[i] * PE);
                const bool live = ((pmask >> i) & 1u) && m < p.m;
#pragma unroll
                for (int t = 0; t < PE / 4; ++t)
                    raw[m][i * (PE / 4) + t] = live ? xp[t] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    }

    __device__ __forceinline__ void unpack_x(const float4 (&raw)[M][8]) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 t = raw[m][i];
                xr[m][4 * i] = t.x; xr[m][4 * i + 1] = t.y; xr[m][4 * i + 2] = t.z; xr[m][4 * i + 3] = t.w;
            }
        }
    }

    __device__ __forceinline__ void issue(int blk, Batch &bt) const {
        const int row0 = blk * L.rpb;
        bt.ok = 0u;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int row_raw = row0 + grp * L.jr + j * L.rps + rr;
            const bool ok = act && row_raw < p.n;
            bt.ok |= ok ? (1u << j) : 0u;
            const int row = !ok ? 0 : (EPI == EPI_ROPE ? rope_row(row_raw, p.rope.hd) : row_raw);
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const uint8_t *w = static_cast<const uint8_t *>(d ? p.w1 : p.w0);
#pragma unroll
                for (int i = 0; i < LD; ++i)
                    bt.q[d][j][i] = load_nt16(w + (size_t)row * bpr + (size_t)piece[i] * 16);
            }
        }
    }

    __device__ __forceinline__ void dots(const Batch &bt, float (&v)[V]) const {
#pragma unroll
        for (int j = 0; j < J; ++j) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                float acc[M];
#pragma unroll
                for (int m = 0; m < M; ++m) acc[m] = 0.f;
                if constexpr (WT == W_I8) {
#pragma unroll
                    for (int i = 0; i < LD; ++i) {
                        const uint32_t dw4[4] = {bt.q[d][j][i].x, bt.q[d][j][i].y, bt.q[d][j][i].z,
                                                 bt.q[d][j][i].w};
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const uint32_t u = dw4[k];
                            const float f[4] = {(float)(int8_t)(u & 0xFFu),
                                                (float)(int8_t)((u >> 8) & 0xFFu),
                                                (float)(int8_t)((u >> 16) & 0xFFu),
                                                (float)(int8_t)(u >> 24)};
#pragma unroll
                            for (int e = 0; e < 4; ++e)
#pragma unroll
                                for (int m = 0; m < M; ++m)
                                    acc[m] = fmaf(f[e], xr[m][16 * i + 4 * k + e], acc[m]);
                        }
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < LD; ++i) {
                        const float f[4] = {__uint_as_float(bt.q[d][j][i].x),
                                            __uint_as_float(bt.q[d][j][i].y),
                                            __uint_as_float(bt.q[d][j][i].z),
                                            __uint_as_float(bt.q[d][j][i].w)};
#pragma unroll
                        for (int e = 0; e < 4; ++e)
#pragma unroll
                            for (int m = 0; m < M; ++m)
                                acc[m] = fmaf(f[e], xr[m][4 * i + e], acc[m]);
                    }
                }
                const bool ok = (bt.ok >> j) & 1u;
#pragma unroll
                for (int m = 0; m < M; ++m) v[(d * J + j) * M + m] = ok ? acc[m] : 0.f;
            }
        }
    }
};

template <int WT, int M, int J, bool DUAL, int EPI>
__global__ __launch_bounds__(512) void k_dense_gemv(DenseParams p, Layout L, Epi e) {
    using G = DenseGemv<WT, M, J, DUAL, EPI>;
    __shared__ float red[kMaxWaves * 64];
    __shared__ EpiShared sh;   // one batch per block: a single LDS set
    G g(p, L);
    typename G::Batch a;
    float4 raw[M][8];
    const int row0 = blockIdx.x * L.rpb;
    const int pos = epi_pos<EPI>(e);
    g.issue_x(raw);
    __builtin_amdgcn_sched_barrier(0);
    g.issue(blockIdx.x, a);
    __builtin_amdgcn_sched_barrier(0);
    const EpiIn in = epi_load<J, M, DUAL, EPI>(L, row0, e, pos);
    __builtin_amdgcn_sched_barrier(0);
    g.unpack_x(raw);
    float v[G::V];
    g.dots(a, v);
    reduce_and_store<G::V, J, M, DUAL, EPI>(v, red, sh, L, g.lane, g.wave, row0, e, in);
}

template <int WT, int M, int J, bool DUAL, int EPI>
int launch(const DenseParams &p, hipStream_t st) {
    constexpr int V = (DUAL ? 2 : 1) * J * M;
    static_assert(V <= 64, "at most 64 partials per lane");
    Layout L;
    const bool prod = p.xw_out || p.ssq_out;
    TB_REQUIRE(make_layout(p.k / 32, Log2<V>::value, J, L, prod ? 16 : 0), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: dense GEMV supports K <= " + std::to_string(kMaxWaves * 64 * 32));
    Epi e{};
    e.b0 = p.b0; e.b1 = p.b1; e.res = p.res; e.y = p.y; e.n = p.n; e.m = p.m;
    e.rs0 = p.rs0; e.rs1 = p.rs1; e.rs0_len = p.rs0_len; e.rs1_len = p.rs1_len;
    e.rope = p.rope;
    e.ssq_in = p.ssq_in; e.ssq_n = p.ssq_n; e.eps = p.eps;
    e.inv_h = p.norm_h > 0 ? 1.0f / (float)p.norm_h : 0.f;
    e.rec_w = p.rec_w; e.xw_out = p.xw_out; e.ssq_out = p.ssq_out;
    e.any = static_cast<const float *>(p.w0);   // n * k / 4 >= n floats (k >= 32)
    if (p.ssq_in)
        TB_REQUIRE(p.m == 1 && p.ssq_n <= kMaxSsqPerThread * L.nwaves * 64, TB_ERR_UNSUPPORTED,
                   "TB_UNSUPPORTED: fused RMSNorm input needs M == 1 and K == H");
    if (prod)
        TB_REQUIRE(p.m == 1 && EPI != EPI_ROPE && L.rpb % 16 == 0 && L.rpb <= kMaxRecRows &&
                       p.n % 32 == 0,
                   TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: fused RMSNorm output needs M == 1, "
                                       "N % 32 == 0 and 16-row blocks");
    if (EPI == EPI_ROPE)
        TB_REQUIRE(p.m == 1 && p.rope.hd % L.rpb == 0 && L.rpb % 2 == 0 && p.n % p.rope.hd == 0,
                   TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: fused RoPE needs whole rotation pairs per block");
    const int grid = (p.n + L.rpb - 1) / L.rpb;
    hipLaunchKernelGGL((k_dense_gemv<WT, M, J, DUAL, EPI>), dim3(grid), dim3(L.nwaves * 64), 0,
                       st, p, L, e);
    TB_LAUNCHED();
    return TB_OK;
}

template <int WT, bool DUAL, int EPI>
int dispatch_m(const DenseParams &p, hipStream_t st) {
    // Rows per block sized for ~16 loads of 16 bytes in flight per lane.
    if constexpr (WT == W_I8) {
        // A fused-RMSNorm producer writes whole 16-row pieces: 16 rows per
        // row group, so the K split over up to 8 waves stays available.
        if (!DUAL && (p.xw_out || p.ssq_out)) return launch<WT, 1, 16, DUAL, EPI>(p, st);
        if (p.m <= 1) return launch<WT, 1, DUAL ? 4 : 8, DUAL, EPI>(p, st);
        return launch<WT, 2, DUAL ? 4 : 8, DUAL, EPI>(p, st);
    } else {
        if (p.m <= 1) return launch<WT, 1, DUAL ? 2 : 4, DUAL, EPI>(p, st);
        return launch<WT, 2, DUAL ? 2 : 4, DUAL, EPI>(p, st);
    }
}

template <int WT>
int dispatch_epi(const DenseParams &p, int epi, hipStream_t st) {
    if (p.w1 != nullptr) return dispatch_m<WT, true, EPI_SWIGLU>(p, st);
    if (epi == EPI_RESID) return dispatch_m<WT, false, EPI_RESID>(p, st);
    if (epi == EPI_ROPE) return launch<WT, 1, WT == W_I8 ? 8 : 4, false, EPI_ROPE>(p, st);
    return dispatch_m<WT, false, EPI_PLAIN>(p, st);
}

}  // namespace

int dense_gemv(const DenseParams &p, int wt, int epi, hipStream_t st) {
    TB_REQUIRE(p.m >= 1 && p.m <= kMaxRowsPerPass, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: dense GEMV pass takes 1..2 rows");
    TB_REQUIRE(!(p.xw_out || p.ssq_out) || (wt == W_I8 && epi == EPI_RESID), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: fused RMSNorm outputs come from INT8 residual projections");
    TB_REQUIRE(p.k % 32 == 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: INT8/FP32 GEMV needs K % 32 == 0, got K=" + std::to_string(p.k));
    if (wt == W_I8) return dispatch_epi<W_I8>(p, epi, st);
    return dispatch_epi<W_F32>(p, epi, st);
}

}  // namespace tb

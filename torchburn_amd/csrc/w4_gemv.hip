// Grouped INT4 (W4A32) GEMV for gfx950: one pass takes 1 or 2 activation rows.
//
// Replaces gemv_w4a32_grouped / gemm_w4a32_grouped (reference
// src/quantization/gemv.rs:1514-1725), the SwiGLU neuron kernels
// (src/quantization/gemv/swiglu.rs:205-289, driven by
// src/quantization/fused_ops.rs:244-407) and the residual add that follows the
// O and down projections (src/llm/decoder.rs:1235-1238, 1344-1347).
//
// Work mapping (one wavefront = 64 lanes):
//   * A row of K elements is cut into chunks of E elements (E/2 bytes of
//     nibbles).  Lane `cl` of wave `ks` owns chunk ks*SW + cl for the whole life
//     of the block, so its slice of x (E floats per activation row) is loaded
//     once into VGPRs and reused for every weight row the block streams.
//   * The K-slices of one row are spread over the KS waves of the block
//     (split-K across wavefronts).  Rows with fewer than 64 chunks share a
//     wave: `rps` rows are processed side by side, one per lane span of 2^b.
//   * Each step the lane issues one coalesced 128-bit load of packed nibbles
//     (E = 32 elements): consecutive lanes read consecutive 16-byte pieces of
//     the same row, so a wave instruction covers 1 KiB of one row.  One f32
//     scale per lane per step (group 32: one per chunk; group 64: one per two).
//   * Unpack in registers: lo = w & 0x0F0F0F0F and hi = w & 0xF0F0F0F0 give
//     eight bytes that v_cvt_f32_ubyte{0..3} turn into n and 16*n.  The odd x
//     elements are pre-divided by 16 (exact) so the high nibble needs no shift,
//     and the "-8" of the stored nibble is applied once per chunk through the
//     precomputed 8 * sum(x_chunk):  sum (n - 8) x = sum n x - 8 sum x.
//   * The per-lane chunk partials of J rows are reduced across the lanes of a
//     row with a transpose-reduction (halving exchanges through ds_bpermute:
//     V values over 64 lanes cost V-1 exchanges instead of 6*V), then across
//     the KS waves through LDS, and the epilogue (bias, residual add, or the
//     SwiGLU silu(g)*u of a gate/up pair) runs on the final sums.
#include "tb_common.hpp"
#include "w4_gemv.hpp"

namespace tb {

namespace {

constexpr int kMaxWaves = 8;   // 512 threads: 256 VGPRs per lane available

template <int N>
struct Log2 {
    static constexpr int value = 1 + Log2<N / 2>::value;
};
template <>
struct Log2<1> {
    static constexpr int value = 0;
};

template <int E>
struct Chunk;
template <>
struct Chunk<32> {
    static constexpr int ndw = 4;
    __device__ static void load(const uint8_t *p, uint32_t (&q)[4]) {
        uint4 v = *reinterpret_cast<const uint4 *>(p);
        q[0] = v.x; q[1] = v.y; q[2] = v.z; q[3] = v.w;
    }
};

// q & mask, opaque to the optimiser.  With the mask visible, the compiler folds
// "(float)((q & 0x0F0F0F0F) >> 8 & 0xFF)" into v_bfe_u32 + v_cvt_f32_ubyte0 (two
// instructions per nibble); behind this AND each byte converts with a single
// v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ uint32_t and_opaque(uint32_t q, uint32_t mask) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(q), "v"(mask));
    return r;
}

// a if !pick_b else b, as bit operations: a plain `pick ? v[i + h] : v[i]` on a
// register array is rewritten by the compiler into a dynamically indexed
// access (a cmp/cndmask chain over the whole array).
__device__ __forceinline__ float select_bits(float a, float b, uint32_t mask_b) {
    return __uint_as_float((__float_as_uint(a) & ~mask_b) | (__float_as_uint(b) & mask_b));
}

// Reduce V per-lane values over the lanes of bits [0, b) of the lane id.
// After the call, lane l holds in v[0] the full sum of value index
// (l >> (b - log2 V)) & (V - 1) over its 2^b-lane span.  Requires V <= 2^b.
template <int V>
__device__ __forceinline__ void transpose_reduce(float (&v)[V], int lane, int b) {
    constexpr int LOGV = Log2<V>::value;
#pragma unroll
    for (int s = 0; s < LOGV; ++s) {
        const int h = (V >> s) >> 1;
        const int mask = 1 << (b - 1 - s);
        const uint32_t up = (lane & mask) ? 0xFFFFFFFFu : 0u;
#pragma unroll
        for (int i = 0; i < h; ++i) {
            const float lo = v[i], hi = v[i + h];
            const float keep = select_bits(lo, hi, up);
            const float send = select_bits(hi, lo, up);
            v[i] = keep + __shfl_xor(send, mask);
        }
    }
    for (int sh = b - LOGV - 1; sh >= 0; --sh) v[0] += __shfl_xor(v[0], 1 << sh);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

template <int M, int E, int J, bool DUAL, int EPI>
__global__ __launch_bounds__(512) void k_w4_gemv(W4Params p) {
    constexpr int D = DUAL ? 2 : 1;
    constexpr int V = D * J * M;
    constexpr int NDW = Chunk<E>::ndw;
    constexpr int LOGV = Log2<V>::value;
    constexpr int OUT = J * M;
    __shared__ float red[kMaxWaves * 64];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nwaves = blockDim.x >> 6;
    const int rr = lane >> p.b;
    const int cl = lane & ((1 << p.b) - 1);
    const int chunk_raw = wave * p.sw + cl;
    const bool act = (cl < p.sw) && (chunk_raw < p.c);
    // Idle lanes read a valid chunk and contribute zero (scale forced to 0).
    const int chunk = act ? chunk_raw : 0;

    // This lane's slice of every activation row, odd elements pre-divided by 16.
    float xr[M][E];
    float xs8[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float sum = 0.f;
        const bool live = act && m < p.m;
        const float4 *xp = reinterpret_cast<const float4 *>(p.x + (size_t)m * p.k + chunk * E);
#pragma unroll
        for (int i = 0; i < E / 4; ++i) {
            float4 t = live ? xp[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            xr[m][4 * i + 0] = t.x;
            xr[m][4 * i + 1] = t.y * 0.0625f;
            xr[m][4 * i + 2] = t.z;
            xr[m][4 * i + 3] = t.w * 0.0625f;
            sum += (t.x + t.y) + (t.z + t.w);
        }
        xs8[m] = 8.0f * sum;
    }

    const int gcols = p.k >> p.gshift;          // scale columns per row
    const int sg = (chunk * E) >> p.gshift;     // this chunk's scale column
    const size_t bpr = (size_t)(p.k >> 1);
    const size_t boff = (size_t)chunk * (E / 2);
    const int nblk = (p.n + p.rows_per_block - 1) / p.rows_per_block;

    for (int blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
        const int row0 = blk * p.rows_per_block;
        // Issue every load of the batch first (J*D 16-byte chunks + scales in
        // flight per lane), then unpack and accumulate.
        uint32_t q[D][J][NDW];
        float sc[D][J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int row_raw = row0 + j * p.rows_per_step + rr;
            const bool ok = act && row_raw < p.n;
            const int row = ok ? row_raw : 0;   // out-of-range rows re-read row 0, weight 0
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const uint8_t *w = d ? p.w1 : p.w0;
                const float *s = d ? p.s1 : p.s0;
                Chunk<E>::load(w + (size_t)row * bpr + boff, q[d][j]);
                const float sv = s[(size_t)row * gcols + sg];
                sc[d][j] = ok ? sv : 0.f;
            }
        }
        __builtin_amdgcn_sched_barrier(0);

        float v[V];
#pragma unroll
        for (int j = 0; j < J; ++j) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                float acc[M];
#pragma unroll
                for (int m = 0; m < M; ++m) acc[m] = 0.f;
#pragma unroll
                for (int dw = 0; dw < NDW; ++dw) {
                    const uint32_t lo = and_opaque(q[d][j][dw], 0x0F0F0F0Fu);
                    const uint32_t hi = and_opaque(q[d][j][dw], 0xF0F0F0F0u);
                    const float f[8] = {(float)(lo & 0xFFu),         (float)(hi & 0xFFu),
                                        (float)((lo >> 8) & 0xFFu),  (float)((hi >> 8) & 0xFFu),
                                        (float)((lo >> 16) & 0xFFu), (float)((hi >> 16) & 0xFFu),
                                        (float)(lo >> 24),           (float)(hi >> 24)};
#pragma unroll
                    for (int e = 0; e < 8; ++e)
#pragma unroll
                        for (int m = 0; m < M; ++m) acc[m] = fmaf(f[e], xr[m][8 * dw + e], acc[m]);
                }
#pragma unroll
                for (int m = 0; m < M; ++m) v[(d * J + j) * M + m] = sc[d][j] * (acc[m] - xs8[m]);
            }
        }

        transpose_reduce<V>(v, lane, p.b);
        const int low = p.b - LOGV;
        if ((cl & ((1 << low) - 1)) == 0) {
            const int idx = (cl >> low) & (V - 1);
            red[(wave * p.rows_per_step + rr) * V + idx] = v[0];
        }
        __syncthreads();

        // Epilogue: one thread per (sub-row, row step, activation row).
        const int t = threadIdx.x;
        if (t < p.rows_per_step * OUT) {
            const int r2 = t / OUT, jm = t - r2 * OUT;
            const int j = jm / M, m = jm - j * M;
            const int row = row0 + j * p.rows_per_step + r2;
            if (row < p.n && m < p.m) {
                float a0 = 0.f, a1 = 0.f;
                for (int w = 0; w < nwaves; ++w) {
                    const float *rw = red + (w * p.rows_per_step + r2) * V;
                    a0 += rw[j * M + m];
                    if (DUAL) a1 += rw[(J + j) * M + m];
                }
                const size_t o = (size_t)m * p.n + row;
                if (EPI == EPI_SWIGLU) {
                    const float g = a0 + (p.b0 ? p.b0[row] : 0.f);
                    const float u = a1 + (p.b1 ? p.b1[row] : 0.f);
                    p.y[o] = silu(g) * u;
                } else {
                    const float val = a0 + (p.b0 ? p.b0[row] : 0.f);
                    p.y[o] = (EPI == EPI_RESID) ? p.res[o] + val : val;
                }
            }
        }
        __syncthreads();   // red is rewritten by the next batch
    }
}

int ceil_log2(int v) {
    int b = 0;
    while ((1 << b) < v) ++b;
    return b;
}

template <int M, int E, int J, bool DUAL, int EPI>
int launch(W4Params p, hipStream_t st) {
    constexpr int V = (DUAL ? 2 : 1) * J * M;
    constexpr int LOGV = Log2<V>::value;
    static_assert(V <= 64, "at most 64 partials per lane");
    p.c = p.k / E;
    int ks, bnat;
    if (p.c <= 64) {
        ks = 1;
        bnat = ceil_log2(p.c);
        p.sw = p.c;
    } else {
        ks = (p.c + 63) / 64;
        bnat = 6;
        p.sw = (p.c + ks - 1) / ks;
    }
    TB_REQUIRE(ks <= kMaxWaves, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: w4a32 GEMV supports K <= " + std::to_string(kMaxWaves * 64 * E));
    p.b = bnat > LOGV ? bnat : LOGV;
    p.rows_per_step = 64 >> p.b;
    p.rows_per_block = J * p.rows_per_step;
    const int nblk = (int)((p.n + p.rows_per_block - 1) / p.rows_per_block);
    const int grid = (nblk + p.batches_per_block - 1) / p.batches_per_block;
    hipLaunchKernelGGL((k_w4_gemv<M, E, J, DUAL, EPI>), dim3(grid), dim3(ks * 64), 0, st, p);
    TB_LAUNCHED();
    return TB_OK;
}

template <bool DUAL, int EPI>
int dispatch_m(const W4Params &p, hipStream_t st) {
    // x stays in VGPRs (32 per activation row), so one pass takes <= 2 rows.
    if (p.m <= 1) return launch<1, 32, DUAL ? 8 : 16, DUAL, EPI>(p, st);
    return launch<2, 32, DUAL ? 4 : 8, DUAL, EPI>(p, st);
}

}  // namespace

int w4_gemv(W4Params p, int epi, hipStream_t st) {
    TB_REQUIRE(p.m >= 1 && p.m <= kMaxRowsPerPass, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: w4 GEMV pass takes 1..2 rows");
    const bool dual = p.w1 != nullptr;
    if (dual) return dispatch_m<true, EPI_SWIGLU>(p, st);
    if (epi == EPI_RESID) return dispatch_m<false, EPI_RESID>(p, st);
    return dispatch_m<false, EPI_PLAIN>(p, st);
}

}  // namespace tb

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
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <>
struct Chunk<32> {
    static constexpr int ndw = 4;
    // Weights are streamed exactly once: non-temporal 128-bit loads keep them
    // from displacing x, scales and partials in L2 / Infinity Cache.
    __device__ static void load(const uint8_t *p, uint32_t (&q)[4]) {
        u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
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
struct W4Gemv {
    static constexpr int D = DUAL ? 2 : 1;
    static constexpr int V = D * J * M;
    static constexpr int NDW = Chunk<E>::ndw;
    static constexpr int LOGV = Log2<V>::value;
    static constexpr int OUT = J * M;

    // One batch of J rows (x D matrices): the raw nibble chunks, the raw scales
    // and a bit per row that is clear for idle lanes and rows past N (their
    // scale is replaced by 0 when the batch is consumed, not when it is issued,
    // so that issuing never waits for a load).
    struct Batch {
        uint32_t q[D][J][NDW];
        float sc[D][J];
        uint32_t ok;
    };

    const W4Params &p;
    int lane, wave, nwaves, rr, cl, chunk;
    bool act;
    size_t bpr, boff;
    int gcols, sg;
    // x chunk as a 24-bit integer per element: x_i ~= sx * X_i, |X_i| < 2^23, sx a
    // power of two,
    // held as U_i = X_i + 2^23 in six 4-bit limbs packed in nibble order
    // (limb[l][d] nibble e = bits [4l, 4l+4) of U_{8d+e}), ready for v_dot8_u32_u4.
    uint32_t limb[M][6][NDW];
    int sxq[M];     // sum_i X_i
    float sx[M];    // dequantisation step of this lane's x chunk
    bool finite;    // false -> the wave takes the f32 path (NaN/Inf propagate)

    __device__ __forceinline__ explicit W4Gemv(const W4Params &pp) : p(pp) {
        lane = threadIdx.x & 63;
        wave = threadIdx.x >> 6;
        nwaves = blockDim.x >> 6;
        rr = lane >> p.b;
        cl = lane & ((1 << p.b) - 1);
        const int chunk_raw = wave * p.sw + cl;
        act = (cl < p.sw) && (chunk_raw < p.c);
        // Idle lanes read a valid chunk and contribute zero (scale forced to 0).
        chunk = act ? chunk_raw : 0;
        gcols = p.k >> p.gshift;
        sg = (chunk * E) >> p.gshift;
        bpr = (size_t)(p.k >> 1);
        boff = (size_t)chunk * (E / 2);
    }

    // The lane's x chunk records (one per activation row), loaded before the
    // weight stream: dot products wait only for them and the batch, never for
    // a later load (loads retire in issue order).
    struct XRec {
        u32x4 limbs[M][6];
        u32x2 tail[M];   // {step bits, sum of integers}; the 2 pad dwords are not read
    };

    __device__ __forceinline__ void issue_x(XRec &xr) const {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const int mm = m < p.m ? m : 0;
            const uint32_t *rp = p.xq + ((size_t)mm * p.c + chunk) * kXRecDwords;
#pragma unroll
            for (int i = 0; i < 6; ++i) xr.limbs[m][i] = reinterpret_cast<const u32x4 *>(rp)[i];
            xr.tail[m] = *reinterpret_cast<const u32x2 *>(rp + 24);
        }
    }

    __device__ __forceinline__ void unpack_x(const XRec &xr) {
        bool fin = true;
#pragma unroll
        for (int m = 0; m < M; ++m) {
#pragma unroll
            for (int l = 0; l < 6; ++l) {
                const u32x4 t = xr.limbs[m][l];
                limb[m][l][0] = t.x; limb[m][l][1] = t.y; limb[m][l][2] = t.z; limb[m][l][3] = t.w;
            }
            sx[m] = __uint_as_float(xr.tail[m].x);
            sxq[m] = (int)xr.tail[m].y;
            fin = fin && (m >= p.m || !__builtin_isnan(sx[m]));
        }
        // One vote per wave, so the integer path runs without per-lane branches.
        finite = __all(fin ? 1 : 0) != 0;
    }

    // f32 chunk dot for a wave whose x holds NaN/Inf: sum (n - 8) * x_i as the
    // reference's unpack-and-fma does, so non-finite values propagate.
    __device__ __forceinline__ float chunk_dot_f32(const uint32_t (&q)[NDW], int m) const {
        const float4 *xp = reinterpret_cast<const float4 *>(p.x + (size_t)m * p.k + chunk * E);
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
        const int row0 = blk * p.rows_per_block;
        bt.ok = 0u;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int row_raw = row0 + j * p.rows_per_step + rr;
            const bool ok = act && row_raw < p.n;
            bt.ok |= ok ? (1u << j) : 0u;
            const int row = ok ? row_raw : 0;   // rows past N re-read row 0 with weight 0
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const uint8_t *w = d ? p.w1 : p.w0;
                const float *s = d ? p.s1 : p.s0;
                Chunk<E>::load(w + (size_t)row * bpr + boff, bt.q[d][j]);
                bt.sc[d][j] = s[(size_t)row * gcols + sg];
            }
        }
    }

    // Unpacks and accumulates batch `blk`, reduces it and runs the epilogue.
    __device__ __forceinline__ void finish(int blk, const Batch &bt, float *red) const {
        // Per chunk: sum_i n_i U_i from six v_dot8_u32_u4 (one per limb) and
        // sum_i n_i from one more against 0x11111111, all exact in u32; then
        //   sum_i (n_i - 8) X_i = 4096 * (hi - 2048 * sum n) + lo - 8 * sum X
        // with lo / hi the limb sums 0..2 / 3..5.  One f32 rounding at the end.
        float v[V];
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
        } else {
#pragma unroll
        for (int j = 0; j < J; ++j) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const uint32_t(&q)[NDW] = bt.q[d][j];
                uint32_t sn = 0u;
#pragma unroll
                for (int dw = 0; dw < NDW; ++dw) sn = __builtin_amdgcn_udot8(q[dw], 0x11111111u, sn, false);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    uint32_t a[6];
#pragma unroll
                    for (int l = 0; l < 6; ++l) {
                        a[l] = 0u;
#pragma unroll
                        for (int dw = 0; dw < NDW; ++dw)
                            a[l] = __builtin_amdgcn_udot8(q[dw], limb[m][l][dw], a[l], false);
                    }
                    const int lo = (int)(a[0] + 16u * a[1] + 256u * a[2]);
                    const int hi = (int)(a[3] + 16u * a[4] + 256u * a[5]);
                    const int t = hi - 2048 * (int)sn;
                    const float r = 8.0f * (float)(512 * t - sxq[m]) + (float)lo;
                    const float sc = ((bt.ok >> j) & 1u) ? bt.sc[d][j] : 0.f;
                    v[(d * J + j) * M + m] = sc * (sx[m] * r);
                }
            }
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
        const int row0 = blk * p.rows_per_block;
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
    }
};

// One block = one batch of rows.  Order matters: x loads, then the batch's
// weight and scale loads, then the limb build (which only waits for x, since
// loads retire in issue order), then the dot products.  Straight-line code, so
// no loop back-edge makes the compiler drain the load counter early.
template <int M, int E, int J, bool DUAL, int EPI>
__global__ __launch_bounds__(512) void k_w4_gemv(W4Params p) {
    using G = W4Gemv<M, E, J, DUAL, EPI>;
    __shared__ float red[kMaxWaves * 64];
    G g(p);
    typename G::Batch a;
    typename G::XRec xr;
    g.issue_x(xr);
    __builtin_amdgcn_sched_barrier(0);
    g.issue(blockIdx.x, a);
    __builtin_amdgcn_sched_barrier(0);
    g.unpack_x(xr);
    g.finish(blockIdx.x, a, red);
}

// Builds the x chunk records read by the GEMV (see kXRecDwords).  Eight
// consecutive lanes share one (activation row, 32-element chunk), four elements
// each.  x_i ~= sx * X_i with sx = 2^(e - 23), amax < 2^e, |X_i| < 2^23: the
// power-of-two step makes the scaling exact and rounds off only bits below
// 2^(e - 23), the precision an f32 partial sum of this chunk has.  Limb l of
// U_i = X_i + 2^23 (bits [4l, 4l + 4)) goes to nibble (i & 7) of dword
// limb[l][i >> 3], the nibble order of the packed weights.
__global__ __launch_bounds__(256) void k_xquant(const float *__restrict__ x,
                                               uint32_t *__restrict__ xq, int m, int k) {
    const int c = k / 32;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int rec = t >> 3, sub = t & 7;
    const bool live = rec < m * c;   // whole 8-lane groups are live or not
    const int row = live ? rec / c : 0, ch = live ? rec - row * c : 0;
    const float4 v = live ? reinterpret_cast<const float4 *>(x + (size_t)row * k + ch * 32)[sub]
                          : make_float4(0.f, 0.f, 0.f, 0.f);
    const float xv[4] = {v.x, v.y, v.z, v.w};
    int fin = 1;
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        fin &= __builtin_isfinite(xv[i]) != 0;
        amax = fmaxf(amax, fabsf(xv[i]));
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, o));
        fin &= __shfl_xor(fin, o);
    }
    int e = 0;
    (void)frexpf(amax, &e);
    e = e < -100 ? -100 : e;
    const float inv = ldexpf(1.0f, 23 - e);
    uint32_t lw[6] = {0u, 0u, 0u, 0u, 0u, 0u};
    int ssum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int X = fin ? (int)rintf(xv[i] * inv) : 0;
        X = X > 8388607 ? 8388607 : (X < -8388607 ? -8388607 : X);
        ssum += X;
        const uint32_t U = (uint32_t)(X + 8388608);
        const int nib = (sub & 1) * 4 + i;   // nibble of element 4*sub + i in its dword
#pragma unroll
        for (int l = 0; l < 6; ++l) lw[l] |= ((U >> (4 * l)) & 15u) << (4 * nib);
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) ssum += __shfl_xor(ssum, o);
#pragma unroll
    for (int l = 0; l < 6; ++l) lw[l] |= __shfl_xor(lw[l], 1);
    if (!live) return;
    uint32_t *o = xq + (size_t)rec * kXRecDwords;
    if ((sub & 1) == 0) {
#pragma unroll
        for (int l = 0; l < 6; ++l) o[l * 4 + (sub >> 1)] = lw[l];
    }
    if (sub == 0) {
        o[24] = __float_as_uint(fin ? ldexpf(1.0f, e - 23) : __builtin_nanf(""));
        o[25] = (uint32_t)ssum;
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
    const int grid = (int)((p.n + p.rows_per_block - 1) / p.rows_per_block);
    hipLaunchKernelGGL((k_w4_gemv<M, E, J, DUAL, EPI>), dim3(grid), dim3(ks * 64), 0, st, p);
    TB_LAUNCHED();
    return TB_OK;
}

template <bool DUAL, int EPI>
int dispatch_m(const W4Params &p, hipStream_t st) {
    // x stays in VGPRs (32 per activation row), so one pass takes <= 2 rows.
    // J (rows per batch) is sized so two batch buffers fit beside x.
    if (p.m <= 1) {
        // Default rows per block: 8 for a gate/up pair (16 loads in flight per
        // lane), 16 for a single matrix.
        const int j = p.rows_j ? p.rows_j : (DUAL ? 8 : 16);
        if (j == 4) return launch<1, 32, 4, DUAL, EPI>(p, st);
        if constexpr (!DUAL) {
            if (j == 16) return launch<1, 32, 16, DUAL, EPI>(p, st);
        }
        return launch<1, 32, 8, DUAL, EPI>(p, st);
    }
    return launch<2, 32, DUAL ? 2 : 4, DUAL, EPI>(p, st);
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
    TB_REQUIRE(p.m >= 1 && p.m <= kMaxRowsPerPass, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: w4 GEMV pass takes 1..2 rows");
    const bool dual = p.w1 != nullptr;
    if (dual) return dispatch_m<true, EPI_SWIGLU>(p, st);
    if (epi == EPI_RESID) return dispatch_m<false, EPI_RESID>(p, st);
    return dispatch_m<false, EPI_PLAIN>(p, st);
}

}  // namespace tb

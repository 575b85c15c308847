// Device helpers shared by the GEMV kernels (INT4 w4_gemv.hip, INT8/FP32
// gemv_dense.hip) and the decoder kernels that produce GEMV inputs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "w4_gemv.hpp"

namespace tb {
namespace gemv {

constexpr int kMaxWaves = 8;   // 512 threads per block: 256 VGPRs per lane available
// 1024-thread blocks (at most 128 VGPRs per lane): more row groups per block
// for kernels whose epilogue needs 16-row blocks
constexpr int kMaxWavesWide = 16;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int N>
struct Log2 {
    static constexpr int value = 1 + Log2<N / 2>::value;
};
template <>
struct Log2<1> {
    static constexpr int value = 0;
};

inline int ceil_log2(int v) {
    int b = 0;
    while ((1 << b) < v) ++b;
    return b;
}

// Streamed-once weights: non-temporal 128-bit loads keep them from displacing
// activations, scales and partials in L2 / Infinity Cache.
__device__ __forceinline__ u32x4 load_nt16(const void *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

// ---- v2 weight stream (34-byte group-64 blocks: 32 bytes of nibbles, then
// the group scale as little-endian IEEE binary16; packed_v2.rs:26-143) ----
constexpr int kV2Block = 34;

// The 16 nibble bytes at byte offset o (o even) of a v2 stream whose base is
// 4-byte aligned.  Five dword-aligned loads cover [o & ~3, (o & ~3) + 20), and
// a funnel shift drops the 0 or 2 leading bytes.  Every dword read holds a
// byte of the chunk or of its block's scale, so no read leaves the buffer.
__device__ __forceinline__ u32x4 load_v2_chunk(const uint8_t *w, uint32_t o) {
    const uint32_t *p = reinterpret_cast<const uint32_t *>(w + (o & ~3u));
    uint32_t d[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) d[i] = __builtin_nontemporal_load(p + i);
    const uint32_t sh = (o & 2u) * 8u;   // 0 or 16 bits
    u32x4 r;
    r.x = __builtin_amdgcn_alignbit(d[1], d[0], sh);
    r.y = __builtin_amdgcn_alignbit(d[2], d[1], sh);
    r.z = __builtin_amdgcn_alignbit(d[3], d[2], sh);
    r.w = __builtin_amdgcn_alignbit(d[4], d[3], sh);
    return r;
}

// binary16 bits -> f32 (packed_v2.rs:32-56) in integer arithmetic, so f16
// subnormal scales decode exactly whatever the denormal mode: exponent 0 is
// m * 2^-24, 31 is inf / NaN, otherwise the exponent is rebiased.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    const float sub = (float)m * 5.9604644775390625e-8f;   // m * 2^-24, exact
    const uint32_t nrm = ((e + 112u) << 23) | (m << 13);
    const uint32_t special = m ? 0x7FC00000u : 0x7F800000u;
    const uint32_t bits = e == 0 ? __float_as_uint(sub) : (e == 31 ? special : nrm);
    return __uint_as_float(e == 31 && m ? bits : (bits | sign));
}

// The f32 scale of the v2 block that starts at byte offset b.
__device__ __forceinline__ float load_v2_scale(const uint8_t *w, uint32_t b) {
    return f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(w + b + 32u));
}

// Non-temporal 16-byte load of 4 floats (streamed-once data such as the KV cache).
__device__ __forceinline__ float4 load_nt_f4(const float *p) {
    typedef float f32x4_t __attribute__((ext_vector_type(4)));
    const f32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t *>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

// q & mask, opaque to the optimiser.  With the mask visible, the compiler folds
// "(float)((q & 0x0F0F0F0F) >> 8 & 0xFF)" into v_bfe_u32 + v_cvt_f32_ubyte0 (two
// instructions per byte); behind this AND each byte converts with a single
// v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ uint32_t and_opaque(uint32_t q, uint32_t mask) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(q), "v"(mask));
    return r;
}

__device__ __forceinline__ uint32_t xor_opaque(uint32_t q, uint32_t mask) {
    uint32_t r;
    asm("v_xor_b32 %0, %1, %2" : "=v"(r) : "v"(q), "v"(mask));
    return r;
}

// a if !pick_b else b, as bit operations: a plain `pick ? v[i + h] : v[i]` on a
// register array is rewritten by the compiler into a dynamically indexed
// access (a cmp/cndmask chain over the whole array).
__device__ __forceinline__ float select_bits(float a, float b, uint32_t mask_b) {
    return __uint_as_float((__float_as_uint(a) & ~mask_b) | (__float_as_uint(b) & mask_b));
}

// v from lane (lane ^ MASK) of the wave, in VALU moves instead of an
// LDS-crossbar permute: quad permutes for 1 and 2, the row shifts by 4 either
// way picked by lane bit 2, a row rotation by 8 (which swaps the row's
// halves), and gfx950's 16- and 32-lane swaps.
template <int MASK>
__device__ __forceinline__ float shfl_xor_c(float v) {
    static_assert(MASK == 1 || MASK == 2 || MASK == 4 || MASK == 8 || MASK == 16 || MASK == 32,
                  "a power of two below 64");
    const int lane = threadIdx.x & 63;
    const int iv = __float_as_int(v);
    if constexpr (MASK == 1) {
        return __int_as_float(__builtin_amdgcn_update_dpp(iv, iv, 0xB1, 0xF, 0xF, false));
    } else if constexpr (MASK == 2) {
        return __int_as_float(__builtin_amdgcn_update_dpp(iv, iv, 0x4E, 0xF, 0xF, false));
    } else if constexpr (MASK == 4) {
        const int up = __builtin_amdgcn_update_dpp(iv, iv, 0x104, 0xF, 0xF, false);   // i + 4
        const int dn = __builtin_amdgcn_update_dpp(iv, iv, 0x114, 0xF, 0xF, false);   // i - 4
        return __int_as_float((lane & 4) ? dn : up);
    } else if constexpr (MASK == 8) {
        return __int_as_float(__builtin_amdgcn_update_dpp(iv, iv, 0x128, 0xF, 0xF, false));
    } else if constexpr (MASK == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap((unsigned)iv, (unsigned)iv, false, false);
        return __uint_as_float((lane & 16) ? r[0] : r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap((unsigned)iv, (unsigned)iv, false, false);
        return __uint_as_float((lane & 32) ? r[0] : r[1]);
    }
}

// The same for a mask known only at run time (wave-uniform; a constant after
// unrolling folds the switch away).
__device__ __forceinline__ float shfl_xor_u(float v, int mask) {
    switch (mask) {
    case 1: return shfl_xor_c<1>(v);
    case 2: return shfl_xor_c<2>(v);
    case 4: return shfl_xor_c<4>(v);
    case 8: return shfl_xor_c<8>(v);
    case 16: return shfl_xor_c<16>(v);
    case 32: return shfl_xor_c<32>(v);
    default: return __shfl_xor(v, mask);
    }
}

// Reduce V per-lane values over the lanes of bits [0, B) of the lane id
// (halving exchanges: V - 1 exchanges for V values instead of log2(64) per
// value).  After the call, lane l holds in v[0] the full sum of value index
// (l >> (B - log2 V)) & (V - 1) over its 2^B-lane span.  Requires V <= 2^B.
template <int V, int B>
__device__ __forceinline__ void transpose_reduce_c(float (&v)[V], int lane) {
    constexpr int LOGV = Log2<V>::value;
    static_assert(LOGV <= B && B <= 6, "V <= 2^B <= 64");
#pragma unroll
    for (int s = 0; s < LOGV; ++s) {
        const int h = (V >> s) >> 1;
        const int mask = 1 << (B - 1 - s);
        const uint32_t up = (lane & mask) ? 0xFFFFFFFFu : 0u;
#pragma unroll
        for (int i = 0; i < h; ++i) {
            const float lo = v[i], hi = v[i + h];
            const float keep = select_bits(lo, hi, up);
            const float send = select_bits(hi, lo, up);
            v[i] = keep + shfl_xor_u(send, mask);
        }
    }
#pragma unroll
    for (int sh = B - LOGV - 1; sh >= 0; --sh) v[0] += shfl_xor_u(v[0], 1 << sh);
}

// transpose_reduce_c for a lane-bit count b known at run time (wave-uniform).
template <int V>
__device__ __forceinline__ void transpose_reduce(float (&v)[V], int lane, int b) {
    constexpr int LOGV = Log2<V>::value;
    switch (b) {
    case 6: transpose_reduce_c<V, 6>(v, lane); break;
    case 5: if constexpr (LOGV <= 5) transpose_reduce_c<V, 5>(v, lane); break;
    case 4: if constexpr (LOGV <= 4) transpose_reduce_c<V, 4>(v, lane); break;
    case 3: if constexpr (LOGV <= 3) transpose_reduce_c<V, 3>(v, lane); break;
    case 2: if constexpr (LOGV <= 2) transpose_reduce_c<V, 2>(v, lane); break;
    case 1: if constexpr (LOGV <= 1) transpose_reduce_c<V, 1>(v, lane); break;
    default: if constexpr (LOGV == 0) transpose_reduce_c<V, 0>(v, lane); break;
    }
}

// silu(g) = g / (1 + exp(-g)), as the reference writes it
// (src/quantization/fused_ops.rs:404-405).
__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// Lane layout of one GEMV block: `nks` K-slices of `sw` chunk-lanes (one wave
// each); a row spans 2^b lanes and `rps` rows are processed side by side per
// step; `ng` row groups of `jr` = J * rps rows each (ng * nks waves in all).
struct Layout {
    int c, sw, b, rps, rpb;   // chunks per row, lanes per slice, log2 span, rows/step, rows/block
    int nks, ng, jr;          // K-slice waves, row groups, rows per group
    int nwaves;
};

// Picks the split of a row of `c` chunks over waves and lanes for V partials
// per lane, with at least `min_rows` rows per block when the wave budget allows
// (row groups).  Returns false when the row needs more than kMaxWaves slices.
inline bool make_layout(int c, int logv, int j, Layout &L, int min_rows = 0,
                        int max_waves = kMaxWaves) {
    int bnat;
    if (c <= 64) {
        L.nks = 1;
        bnat = ceil_log2(c);
        L.sw = c;
    } else {
        L.nks = (c + 63) / 64;
        bnat = 6;
        L.sw = (c + L.nks - 1) / L.nks;
    }
    if (L.nks > kMaxWaves) return false;
    L.c = c;
    L.b = bnat > logv ? bnat : logv;
    L.rps = 64 >> L.b;
    L.jr = j * L.rps;
    L.ng = 1;
    while (L.jr * L.ng < min_rows && L.nks * L.ng * 2 <= max_waves) L.ng *= 2;
    L.nwaves = L.nks * L.ng;
    L.rpb = L.jr * L.ng;
    return true;
}

// Rotation-pair order of the rows of a head: logical rows 2i and 2i+1 of head
// h are physical rows h*hd + i and h*hd + i + hd/2.
__device__ __forceinline__ int rope_row(int l, int hd) {
    const int head = l / hd, r = l - head * hd, i = r >> 1;
    return head * hd + ((r & 1) ? i + (hd >> 1) : i);
}

// Output side of a GEMV block.  Row scales (per-channel INT8) multiply the row
// dot before bias: y = dot * s + b, as the reference's w8a32 rows do
// (src/quantization/gemv.rs:777-785).
//
// Fused RMSNorm (decoder, M == 1).  A consumer whose records hold x * w_norm
// (not yet divided by the RMS) gets `ssq_in`: sums of squares of x over
// consecutive 16-element pieces.  Every block sums them in the same order and
// scales its dots by inv = 1 / sqrt(sum / H + eps) (fast_rms_norm,
// src/quantization/fused_ops.rs:1066-1089).  A producer whose rows form x (the
// O and down projections with the residual add) or h (gate/up) writes, besides
// y, the records of y * rec_w (rec_w = the next RMSNorm weight, or none) and,
// with `ssq_out`, the 16-element sums of squares of y.
struct Epi {
    const float *b0, *b1;     // bias of the (first, second) matrix or null
    const float *rs0, *rs1;   // per-row scales or null; *_len == 1 -> one scalar
    int rs0_len, rs1_len;
    const float *res;         // residual [m, n] for EPI_RESID
    float *y;                 // output [m, n]
    int n, m;
    RopeArgs rope;            // EPI_ROPE (m == 1)
    const float *ssq_in;      // consumer: [ssq_n] sums of squares, or null
    int ssq_n;
    float inv_h, eps;         // 1 / H and the RMSNorm epsilon
    uint32_t *rec_out;        // producer: records of y [* rec_w], or null
    const float *rec_w;
    float *xw_out;            // producer: y [* rec_w] in f32 (the consumer's NaN/Inf path)
    float *ssq_out;           // producer: [n / 16] sums of squares of y, or null
    const float *any;         // >= n readable floats: stand-in base for absent operands
};

__device__ __forceinline__ float row_scale(const float *rs, int len, int row) {
    return rs ? (len > 1 ? rs[row] : rs[0]) : 1.0f;
}

// Sums of squares per thread of a fused-RMSNorm consumer: the consumer's K is H,
// so its block has 64 * ceil(H / 2048) threads or more and H / 16 entries to sum.
constexpr int kMaxSsqPerThread = 2;

// Epilogue operands of one output (row, activation row): loaded by the thread
// that will write it right after the weight loads are issued, so they arrive
// while the dot products run instead of costing a round trip after the
// reduction.
struct EpiIn {
    float b0, b1, s0, s1;   // bias and row scale (1 when none) of the row (and its pair)
    float res;              // residual (EPI_RESID)
    float pb0, ps0;         // EPI_ROPE: bias and scale of the rotation partner row
    float c, s;             // EPI_ROPE: cos / sin at the current position
    float ssq[kMaxSsqPerThread];   // this thread's share of the fused-RMSNorm sums of squares
    int pos;                // EPI_ROPE
};

// Output slot of thread t: row group g = t / (rps * J * M), then (r2, j, m)
// inside the group; the row is row0 + g * jr + j * rps + r2.  False for idle
// threads and rows past n / m.
template <int J, int M>
__device__ __forceinline__ bool epi_slot(const Layout &L, int row0, const Epi &e, int &row, int &m,
                                         int &grp, int &j, int &r2) {
    constexpr int OUT = J * M;
    const int t = threadIdx.x;
    const int per = L.rps * OUT;
    grp = j = r2 = m = 0;
    row = row0;
    if (t >= L.ng * per) return false;
    grp = t / per;
    const int tt = t - grp * per;
    r2 = tt / OUT;
    const int jm = tt - r2 * OUT;
    j = jm / M;
    m = jm - j * M;
    row = row0 + grp * L.jr + j * L.rps + r2;
    return row < e.n && m < e.m;
}

// EPI_ROPE: the position, first of all loads (the cos / sin loads need it).
template <int EPI>
__device__ __forceinline__ int epi_pos(const Epi &e) {
    return EPI == EPI_ROPE ? *e.rope.pos : 0;
}

// Every load is unconditional (clamped indices, the `any` buffer standing in
// for absent operands) and the raw values are fixed up only in the epilogue
// (epi_fix): with per-lane branches or a value consumed here, the compiler
// would wait for every weight load issued before these before the dot
// products could start.
template <int J, int M, bool DUAL, int EPI>
__device__ __forceinline__ EpiIn epi_load(const Layout &L, int row0, const Epi &e, int pos) {
    EpiIn in;
    in.b0 = in.b1 = in.res = in.pb0 = in.c = in.s = 0.f;
    in.s0 = in.s1 = in.ps0 = 1.f;
    in.pos = pos;
    {
        const float *sq = e.ssq_in ? e.ssq_in : e.any;   // summed only with ssq_in
        const int nt = L.nwaves * 64;
#pragma unroll
        for (int u = 0; u < kMaxSsqPerThread; ++u) {
            const int i = threadIdx.x + u * nt;
            in.ssq[u] = sq[i < e.ssq_n ? i : 0];
        }
    }
    int row, m, grp, j, r2;
    const bool live = epi_slot<J, M>(L, row0, e, row, m, grp, j, r2);
    const int rw = live ? row : 0, mm = live ? m : 0;
    const float *b0 = e.b0 ? e.b0 : e.any, *b1 = e.b1 ? e.b1 : e.any;
    const float *rs0 = e.rs0 ? e.rs0 : e.any, *rs1 = e.rs1 ? e.rs1 : e.any;
    if (EPI == EPI_ROPE) {
        const RopeArgs &R = e.rope;
        const int prow = rope_row(rw, R.hd), qrow = rope_row(rw ^ 1, R.hd);
        in.b0 = b0[prow];
        in.pb0 = b0[qrow];
        in.s0 = rs0[e.rs0_len > 1 ? prow : 0];
        in.ps0 = rs0[e.rs0_len > 1 ? qrow : 0];
        // cos / sin of the row's place in its head (unused for V rows)
        const int r = prow % R.hd;
        in.c = R.cos_t[(size_t)pos * R.tab_stride + r];
        in.s = R.sin_t[(size_t)pos * R.tab_stride + r];
    } else {
        in.b0 = b0[rw];
        in.s0 = rs0[e.rs0_len > 1 ? rw : 0];
        if (DUAL) {
            in.b1 = b1[rw];
            in.s1 = rs1[e.rs1_len > 1 ? rw : 0];
        }
        if (EPI == EPI_RESID) in.res = e.res[(size_t)mm * e.n + rw];
    }
    return in;
}

// The loaded operands with the absent ones replaced: bias 0, row scale 1.
__device__ __forceinline__ EpiIn epi_fix(EpiIn in, const Epi &e) {
    if (!e.b0) in.b0 = in.pb0 = 0.f;
    if (!e.b1) in.b1 = 0.f;
    if (!e.rs0) in.s0 = in.ps0 = 1.f;
    if (!e.rs1) in.s1 = 1.f;
    return in;
}

// Lane exchanges inside a quad of 4 lanes (DPP quad_perm; every lane of the
// quad must be active): value of lane ^ 1, lane ^ 2.
__device__ __forceinline__ int quad_xor1(int v) {
    return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
}
__device__ __forceinline__ int quad_xor2(int v) {
    return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
}

__device__ __forceinline__ void build_half_rec4(float4 v, int q, bool live, uint32_t *row, int nc,
                                                int chunk, int half);

// LDS a GEMV block needs besides the partials: wave sums of squares, and the
// block's outputs while their records are built.
constexpr int kMaxRecRows = 256;
struct EpiShared {
    float ssq[kMaxWavesWide];
    float out[kMaxRecRows];
};

// Cross-lane + cross-wave reduction of the V = D*J*M per-lane partials and the
// epilogue.  Value index of a partial: (d * J + j) * M + m.
template <int V, int J, int M, bool DUAL, int EPI>
__device__ __forceinline__ void reduce_and_store(float (&v)[V], float *red, EpiShared &sh,
                                                 const Layout &L, int lane, int wave, int row0,
                                                 const Epi &e, const EpiIn &in_raw) {
    constexpr int LOGV = Log2<V>::value;
    const int rr = lane >> L.b;
    const int cl = lane & ((1 << L.b) - 1);
    transpose_reduce<V>(v, lane, L.b);
    const int low = L.b - LOGV;
    if ((cl & ((1 << low) - 1)) == 0) {
        const int idx = (cl >> low) & (V - 1);
        red[(wave * L.rps + rr) * V + idx] = v[0];
    }
    if (e.ssq_in) {
        float t = 0.f;
        const int nt = L.nwaves * 64;
#pragma unroll
        for (int u = 0; u < kMaxSsqPerThread; ++u)
            if ((int)threadIdx.x + u * nt < e.ssq_n) t += in_raw.ssq[u];
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) t += shfl_xor_u(t, o);
        if (lane == 0) sh.ssq[wave] = t;
    }
    __syncthreads();
    float inv = 1.f;
    if (e.ssq_in) {
        float tot = 0.f;
        for (int w = 0; w < L.nwaves; ++w) tot += sh.ssq[w];
        inv = 1.0f / sqrtf(tot * e.inv_h + e.eps);
    }
    int row, m, grp, j, r2;
    const bool live = epi_slot<J, M>(L, row0, e, row, m, grp, j, r2);
    const EpiIn in = epi_fix(in_raw, e);
    float outv = 0.f;
    if (live) {
        float a0 = 0.f, a1 = 0.f;
        for (int ks = 0; ks < L.nks; ++ks) {
            const float *rw = red + ((grp * L.nks + ks) * L.rps + r2) * V;
            a0 += rw[j * M + m];
            if (DUAL) a1 += rw[(J + j) * M + m];
        }
        a0 *= inv;
        a1 *= inv;
        const size_t o = (size_t)m * e.n + row;
        if (EPI == EPI_ROPE) {
            // Both rows of the rotation pair are in this block: logical rows lr
            // and lr ^ 1 (RoPE: src/llm/decoder.rs:28-68, products rounded
            // separately; KV append: decoder.rs:1137-1146).
            const RopeArgs &R = e.rope;
            const int loc = (row ^ 1) - row0;
            const int pg = loc / L.jr, rem = loc - pg * L.jr;
            const int pj = rem / L.rps, pr2 = rem - pj * L.rps;
            float ap = 0.f;
            for (int ks = 0; ks < L.nks; ++ks)
                ap += red[((pg * L.nks + ks) * L.rps + pr2) * V + pj * M];
            ap *= inv;
            const int prow = rope_row(row, R.hd);
            const float own = a0 * in.s0 + in.b0;
            const float oth = ap * in.ps0 + in.pb0;
            const int head = prow / R.hd, r = prow - head * R.hd, half = R.hd >> 1;
            float val = own;
            if (head < R.hq + R.hkv) {
                // r < half: own = x1, oth = x2 -> x1*c - x2*s; else own = x2 -> x2*c + x1*s
                val = r < half ? __fsub_rn(__fmul_rn(own, in.c), __fmul_rn(oth, in.s))
                               : __fadd_rn(__fmul_rn(own, in.c), __fmul_rn(oth, in.s));
            }
            if (head < R.hq) {
                e.y[prow] = val;
            } else if (head < R.hq + R.hkv) {
                R.kc[((size_t)(head - R.hq) * R.max_seq + in.pos) * R.hd + r] = val;
            } else {
                R.vc[((size_t)(head - R.hq - R.hkv) * R.max_seq + in.pos) * R.hd + r] = val;
            }
        } else if (EPI == EPI_SWIGLU) {
            const float g = a0 * in.s0 + in.b0;
            const float u = a1 * in.s1 + in.b1;
            outv = silu(g) * u;
            e.y[o] = outv;
        } else {
            const float val = a0 * in.s0 + in.b0;
            outv = (EPI == EPI_RESID) ? in.res + val : val;
            e.y[o] = outv;
        }
    }
    if (EPI != EPI_ROPE && (e.rec_out || e.xw_out || e.ssq_out)) {
        // Records, y * rec_w in f32 and sums of squares of this block's
        // outputs, M == 1: quads of lanes take one 16-row half each.
        const int t = threadIdx.x;
        // For M == 1 the slots of threads 0 .. rpb-1 are the rpb rows of the block.
        if (t < L.rpb) sh.out[row - row0] = live ? outv : 0.f;
        __syncthreads();
        if (t < (L.rpb >> 2)) {
            const int base = row0 + 16 * (t >> 2), q = t & 3;
            const bool ok = base < e.n;
            const float4 yv = *reinterpret_cast<const float4 *>(&sh.out[4 * t]);
            float4 wv = make_float4(1.f, 1.f, 1.f, 1.f);
            if (ok && e.rec_w) wv = *reinterpret_cast<const float4 *>(e.rec_w + base + 4 * q);
            const float4 xv = make_float4(yv.x * wv.x, yv.y * wv.y, yv.z * wv.z, yv.w * wv.w);
            if (e.rec_out)
                build_half_rec4(xv, q, ok, e.rec_out, e.n >> 5, base >> 5, (base >> 4) & 1);
            if (ok && e.xw_out) *reinterpret_cast<float4 *>(e.xw_out + base + 4 * q) = xv;
            if (e.ssq_out) {
                float sq = fmaf(yv.x, yv.x, fmaf(yv.y, yv.y, fmaf(yv.z, yv.z, yv.w * yv.w)));
                sq += __shfl_xor(sq, 1);
                sq += __shfl_xor(sq, 2);
                if (ok && q == 0) e.ssq_out[base >> 4] = sq;
            }
        }
    }
}

// Builds one half (16 elements) of an x chunk record in a quad of 4
// consecutive lanes; lane q (0..3) holds elements 4q .. 4q + 3 of the half in v.
// x_i ~= sx * X_i with sx = 2^(e - 22), amax < 2^e, |X_i| <= 2^22: the
// power-of-two step makes the scaling exact and rounds off only bits below
// 2^(e - 23), about the precision an f32 partial sum of these elements has.
// X_i is written as six signed base-16 digits d_l in [-8, 7] (X_i = sum_l
// 16^l d_l; six digits reach +-8947848 > 2^22): digit l of X is nibble l of
// X + 0x888888 minus 8, and its 4-bit two's complement that nibble XOR 8, so
// the digit planes are the nibble planes of U_i = (X_i + 0x888888) ^ 0x888888.
// Digit l of element i goes to nibble (i & 7) of dword limb[l][i >> 3] (i =
// element index in the 32-element chunk), the nibble order of the packed
// weights.  A record (kXRecDwords) is 7 quads of 4 dwords: quad l < 6 holds
// digit plane l (dwords 0-1 half 0, 2-3 half 1), quad 6 {step of half 0, step
// of half 1, 0, 0}; a step is NaN when its half holds NaN/Inf.  The records of
// a row of nc chunks are stored by quad: quad i of chunk c at
// row + (i * nc + c) * 4, so a GEMV wave, one chunk per lane, reads each quad
// of 64 consecutive chunks as one contiguous KiB.  All 4 lanes must call this;
// the record of `chunk` is written when `live`.
__device__ __forceinline__ void build_half_rec4(float4 v, int q, bool live, uint32_t *row, int nc,
                                                int chunk, int half) {
    const float xv[4] = {v.x, v.y, v.z, v.w};
    int fin = 1;
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        fin &= __builtin_isfinite(xv[i]) != 0;
        amax = fmaxf(amax, fabsf(xv[i]));
    }
    amax = fmaxf(amax, __int_as_float(quad_xor1(__float_as_int(amax))));
    amax = fmaxf(amax, __int_as_float(quad_xor2(__float_as_int(amax))));
    fin &= quad_xor1(fin);
    fin &= quad_xor2(fin);
    int e = 0;
    (void)frexpf(amax, &e);
    e = e < -100 ? -100 : e;
    const float inv = ldexpf(1.0f, 22 - e);
    uint32_t lw[6] = {0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int X = fin ? (int)rintf(xv[i] * inv) : 0;
        X = X > 4194304 ? 4194304 : (X < -4194304 ? -4194304 : X);
        const uint32_t U = (uint32_t)(X + 0x888888) ^ 0x888888u;
        const int nib = (q & 1) * 4 + i;   // nibble of element 4q + i in its dword
#pragma unroll
        for (int l = 0; l < 6; ++l) lw[l] |= ((U >> (4 * l)) & 15u) << (4 * nib);
    }
#pragma unroll
    for (int l = 0; l < 6; ++l) lw[l] |= (uint32_t)quad_xor1((int)lw[l]);
    if (!live) return;
    uint32_t *rec = row + (size_t)chunk * 4;
    const size_t quad = (size_t)nc * 4;   // dwords between quads of one record
    if ((q & 1) == 0) {
#pragma unroll
        for (int l = 0; l < 6; ++l) rec[l * quad + half * 2 + (q >> 1)] = lw[l];
    }
    if (q == 0) {
        rec[6 * quad + half] = __float_as_uint(fin ? ldexpf(1.0f, e - 22) : __builtin_nanf(""));
        rec[6 * quad + 2 + half] = 0u;
    }
}

// One whole chunk record from 8 consecutive lanes; lane `sub` (0..7) holds
// elements 4*sub .. 4*sub + 3 of chunk `chunk` of a row of nc chunks.
__device__ __forceinline__ void build_xrec8(float4 v, int sub, bool live, uint32_t *row, int nc,
                                            int chunk) {
    build_half_rec4(v, sub & 3, live, row, nc, chunk, sub >> 2);
}

// The six digit-plane dwords of 8 consecutive elements (U[e] of
// build_half_rec4, 24 bits): out[l] nibble e = bits [4l, 4l + 4) of U[e].
// Pairs of elements first merge into bytes (pe: even planes, po: odd planes;
// byte b of pair p holds plane 2b or 2b + 1 of elements 2p, 2p + 1), then
// v_perm_b32 gathers byte b of the four pairs into one dword: 42 VALU
// operations instead of 96 nibble inserts.
__device__ __forceinline__ void pack_limbs8(const uint32_t *U, uint32_t (&out)[6]) {
    uint32_t pe[4], po[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        pe[p] = (U[2 * p] & 0x0F0F0Fu) | ((U[2 * p + 1] << 4) & 0xF0F0F0u);
        po[p] = ((U[2 * p] >> 4) & 0x0F0F0Fu) | (U[2 * p + 1] & 0xF0F0F0u);
    }
#pragma unroll
    for (int b = 0; b < 3; ++b) {
        // selector bytes: b picks byte b of the second operand, 4 + b of the
        // first, 0x0c a zero byte
        const uint32_t slo = 0x0c0c0000u | ((4u + b) << 8) | (uint32_t)b;
        const uint32_t shi = ((4u + b) << 24) | ((uint32_t)b << 16) | 0x0c0cu;
        out[2 * b] = __builtin_amdgcn_perm(pe[1], pe[0], slo) | __builtin_amdgcn_perm(pe[3], pe[2], shi);
        out[2 * b + 1] =
            __builtin_amdgcn_perm(po[1], po[0], slo) | __builtin_amdgcn_perm(po[3], po[2], shi);
    }
}

// The record of one whole chunk (x[e], e = 0..31) built by a single lane, in
// registers: the values build_half_rec4 stores, limb[l][d] = dword d of digit
// plane l, step[h] the step of half h.
__device__ __forceinline__ void lane_chunk_rec(const float (&x)[32], uint32_t (&limb)[6][4],
                                               float (&step)[2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        bool fin = true;
        float amax = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            fin = fin && __builtin_isfinite(x[16 * h + j]);
            amax = fmaxf(amax, fabsf(x[16 * h + j]));
        }
        int e = 0;
        (void)frexpf(amax, &e);
        e = e < -100 ? -100 : e;
        const float inv = ldexpf(1.0f, 22 - e);
        uint32_t U[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            int X = fin ? (int)rintf(x[16 * h + j] * inv) : 0;
            X = X > 4194304 ? 4194304 : (X < -4194304 ? -4194304 : X);
            U[j] = (uint32_t)(X + 0x888888) ^ 0x888888u;
        }
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            uint32_t o[6];
            pack_limbs8(U + 8 * d, o);
#pragma unroll
            for (int l = 0; l < 6; ++l) limb[l][2 * h + d] = o[l];
        }
        step[h] = fin ? ldexpf(1.0f, e - 22) : __builtin_nanf("");
    }
}

}  // namespace gemv
}  // namespace tb

// Single-token decoder-step kernels for gfx950: everything in the reference's
// RustQwenDecoder::step_internal (src/llm/decoder.rs:1051-1374) except the
// GEMVs (w4_gemv.hip, gemv_dense.hip).
//
// All kernels read the token id and position from a small device state block
// (DecState), so one captured hipGraph serves every step, and the greedy argmax
// writes the next token and advances the position on the device.
#include <float.h>

#include <algorithm>

#include "decode.hpp"
#include "gemv_common.hpp"
#include "tb_common.hpp"

namespace tb {

using namespace gemv;

namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += shfl_xor_u(v, o);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, shfl_xor_u(v, o));
    return v;
}

// Block-wide sum; every thread gets the total.  `scratch` holds >= 16 floats.
__device__ __forceinline__ float block_sum(float v, float *scratch) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_sum(v);
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int w = 0; w < nw; ++w) t += scratch[w];
    __syncthreads();
    return t;
}

// x = embed[token] (when embed != null), then
//   xn = (x * (1 / sqrt(sum(x^2) / H + eps))) * w
// (fast_rms_norm, src/quantization/fused_ops.rs:1066-1089; the AVX-512 tier's
// x * inv_rms * w order), and the chunk records of xn for the next INT4 GEMV.
// Each block recomputes the whole sum of squares (H floats from L2, the same
// order in every block, so every block gets the same inverse) and normalises
// and records kNormChunks 32-element chunks of its own.
__global__ __launch_bounds__(256) void k_rmsnorm(const DecState *__restrict__ st,
                                                 const float *__restrict__ embed,
                                                 float *__restrict__ x,
                                                 const float *__restrict__ w,
                                                 float *__restrict__ xn,
                                                 uint32_t *__restrict__ xq, int H, float eps) {
    __shared__ float scratch[16];
    const int tid = threadIdx.x;
    const float *src = embed ? embed + (size_t)st->token * H : x;
    const float4 *s4 = reinterpret_cast<const float4 *>(src);
    float ss = 0.f;
    for (int i = tid; i < H / 4; i += blockDim.x) {
        const float4 v = s4[i];
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
    }
    const float tot = block_sum(ss, scratch);
    const float rms = sqrtf(tot / (float)H + eps);
    const float inv = 1.0f / rms;
    const int c = H / 32;
    const int rec = blockIdx.x * kNormChunks + (tid >> 3), sub = tid & 7;
    const bool live = rec < c && (tid >> 3) < kNormChunks;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) {
        const int i4 = rec * 8 + sub;
        const float4 v = s4[i4];
        if (embed) reinterpret_cast<float4 *>(x)[i4] = v;
        const float4 ww = reinterpret_cast<const float4 *>(w)[i4];
        o.x = __fmul_rn(__fmul_rn(v.x, inv), ww.x);
        o.y = __fmul_rn(__fmul_rn(v.y, inv), ww.y);
        o.z = __fmul_rn(__fmul_rn(v.z, inv), ww.z);
        o.w = __fmul_rn(__fmul_rn(v.w, inv), ww.w);
        reinterpret_cast<float4 *>(xn)[i4] = o;
    }
    if (xq) build_xrec8(o, sub, live, xq, c, live ? rec : 0);
}

// First input of the fused-RMSNorm step: x = embed[token], x * w in f32 and as
// chunk records (w = the first layer's input-norm weight; the consumer divides
// by the RMS) and the sums of squares of x over 16-element pieces.  Eight lanes
// per 32-element chunk.
__global__ __launch_bounds__(256) void k_embed_rec(const DecState *__restrict__ st,
                                                   const float *__restrict__ embed,
                                                   float *__restrict__ x,
                                                   const float *__restrict__ w,
                                                   float *__restrict__ xw,
                                                   uint32_t *__restrict__ xq,
                                                   float *__restrict__ ssq, int H) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int rec = t >> 3, sub = t & 7;
    const bool live = rec < H / 32;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f), ww = make_float4(1.f, 1.f, 1.f, 1.f);
    if (live) {
        const int i4 = rec * 8 + sub;
        v = reinterpret_cast<const float4 *>(embed + (size_t)st->token * H)[i4];
        reinterpret_cast<float4 *>(x)[i4] = v;
        ww = reinterpret_cast<const float4 *>(w)[i4];
    }
    const float4 p = make_float4(v.x * ww.x, v.y * ww.y, v.z * ww.z, v.w * ww.w);
    if (live) reinterpret_cast<float4 *>(xw)[rec * 8 + sub] = p;
    build_xrec8(p, sub, live, xq, H / 32, live ? rec : 0);
    float sq = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, v.w * v.w)));
    sq += __shfl_xor(sq, 1);
    sq += __shfl_xor(sq, 2);
    if (live && (sub & 3) == 0) ssq[rec * 2 + (sub >> 2)] = sq;
}

// Rotate-half RoPE on the q and k heads of qkv and the KV-cache append at the
// current position (src/llm/decoder.rs:28-68, 1115-1146):
//   x1' = x1*c1 - x2*s1,  x2' = x2*c2 + x1*s2   (products rounded separately)
// Block b < hq rotates q head b in place; hq <= b < hq+hkv rotates k head
// b - hq into the cache; the rest copy v heads.  blockDim = hd / 2.
__global__ void k_rope_kv(const DecState *__restrict__ st, float *__restrict__ qkv,
                          const float *__restrict__ cos_t, const float *__restrict__ sin_t,
                          float *__restrict__ kc, float *__restrict__ vc, int hq, int hkv, int hd,
                          int max_seq) {
    const int b = blockIdx.x, i = threadIdx.x, half = hd / 2;
    const int pos = st->pos;
    const float *cp = cos_t + (size_t)pos * hd, *sp = sin_t + (size_t)pos * hd;
    if (b < hq + hkv) {
        float *head = qkv + (size_t)b * hd;
        const float x1 = head[i], x2 = head[i + half];
        const float o1 = __fsub_rn(__fmul_rn(x1, cp[i]), __fmul_rn(x2, sp[i]));
        const float o2 = __fadd_rn(__fmul_rn(x2, cp[i + half]), __fmul_rn(x1, sp[i + half]));
        if (b < hq) {
            head[i] = o1;
            head[i + half] = o2;
        } else {
            float *dst = kc + ((size_t)(b - hq) * max_seq + pos) * hd;
            dst[i] = o1;
            dst[i + half] = o2;
        }
    } else {
        const int h = b - hq - hkv;
        const float *src = qkv + (size_t)(hq + hkv + h) * hd;
        float *dst = vc + ((size_t)h * max_seq + pos) * hd;
        dst[i] = src[i];
        dst[i + half] = src[i + half];
    }
}

// Split-KV decode attention (flash-decoding), one block per (kv head, tile of
// kAttnTile positions), all G = hq/hkv query heads of the group together so
// each K/V row is read from HBM once.  The tile of K and V is loaded into
// registers (every load in flight at once), then staged through LDS; scores
// s = (q . k_t) * (1/sqrt(hd)); per head the tile's max m, l = sum exp(s - m)
// and o = sum exp(s - m) v_t go to `part` ([hq][nsplit][hd + 4], o then m, l).
// Math of the reference: src/llm/decoder.rs:1148-1213.  (A last-block merge
// inside this kernel was measured slower: the device-scope fence every block
// needs before the hand-off writes back its XCD's L2.)
template <int HD>
__global__ __launch_bounds__(256) void k_attn(const DecState *__restrict__ st,
                                              const float *__restrict__ qkv,
                                              const float *__restrict__ kc,
                                              const float *__restrict__ vc,
                                              float *__restrict__ part, int hq, int hkv,
                                              int max_seq, int nsplit, float scale, int cap) {
    constexpr int T = kAttnTile, KP = HD + 4, C4 = HD / 4;
    constexpr int NV = T * C4 / 256;   // float4 of K (and of V) per thread
    static_assert(T <= 64 && NV >= 1, "tile of at most one wave of positions");
    extern __shared__ float sm[];
    const int kvh = blockIdx.x, sp = blockIdx.y, tid = threadIdx.x;
    const int G = hq / hkv;
    const int seq = min(st->pos + 1, cap);
    const int t0 = sp * T;
    if (t0 >= seq) return;   // tile past the sequence: the merge never reads it
    const int tn = min(T, seq - t0);
    float *sq = sm;                 // [G][HD]
    float *sk = sq + G * HD;        // [T][KP]
    float *sv = sk + T * KP;        // [T][HD]
    float *ss = sv + T * HD;        // [G][T]
    float *sml = ss + G * T;        // [G][2]
    const size_t rec = HD + 4;

    const float4 *kb = reinterpret_cast<const float4 *>(kc + ((size_t)kvh * max_seq + t0) * HD);
    const float4 *vb = reinterpret_cast<const float4 *>(vc + ((size_t)kvh * max_seq + t0) * HD);
    float4 kr[NV], vr[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int idx = tid + i * 256;
        const bool ok = idx / C4 < tn;
        kr[i] = ok ? kb[idx] : make_float4(0.f, 0.f, 0.f, 0.f);
        vr[i] = ok ? vb[idx] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int i = tid; i < G * HD; i += blockDim.x) sq[i] = qkv[(size_t)kvh * G * HD + i];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int idx = tid + i * 256;
        const int r = idx / C4, c = idx - r * C4;
        *reinterpret_cast<float4 *>(sk + r * KP + 4 * c) = kr[i];
        *reinterpret_cast<float4 *>(sv + r * HD + 4 * c) = vr[i];
    }
    __syncthreads();
    for (int i = tid; i < G * T; i += blockDim.x) {
        const int g = i / T, t = i - g * T;
        float s = -FLT_MAX;
        if (t < tn) {
            const float4 *qa = reinterpret_cast<const float4 *>(sq + g * HD);
            const float4 *ka = reinterpret_cast<const float4 *>(sk + t * KP);
            float d0 = 0.f, d1 = 0.f;
#pragma unroll
            for (int c = 0; c < C4; c += 2) {
                const float4 a = qa[c], b = ka[c], a2 = qa[c + 1], b2 = ka[c + 1];
                d0 = fmaf(a.x, b.x, fmaf(a.y, b.y, fmaf(a.z, b.z, fmaf(a.w, b.w, d0))));
                d1 = fmaf(a2.x, b2.x, fmaf(a2.y, b2.y, fmaf(a2.z, b2.z, fmaf(a2.w, b2.w, d1))));
            }
            s = (d0 + d1) * scale;
        }
        ss[i] = s;
    }
    __syncthreads();
    const int lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
    for (int g = wave; g < G; g += nw) {
        const float s = lane < T ? ss[g * T + lane] : -FLT_MAX;
        const float m = wave_max(s);
        const float p = lane < tn ? expf(s - m) : 0.f;
        const float l = wave_sum(p);
        if (lane < T) ss[g * T + lane] = p;
        if (lane == 0) {
            sml[2 * g] = m;
            sml[2 * g + 1] = l;
        }
    }
    __syncthreads();
    for (int i = tid; i < G * HD; i += blockDim.x) {
        const int g = i / HD, d = i - g * HD;
        const float *pg = ss + g * T;
        float a0 = 0.f, a1 = 0.f;
        int t = 0;
        for (; t + 1 < tn; t += 2) {
            a0 = fmaf(pg[t], sv[t * HD + d], a0);
            a1 = fmaf(pg[t + 1], sv[(t + 1) * HD + d], a1);
        }
        if (t < tn) a0 = fmaf(pg[t], sv[t * HD + d], a0);
        float *o = part + ((size_t)(kvh * G + g) * nsplit + sp) * rec;
        o[d] = a0 + a1;
        if (d == 0) {
            o[HD] = sml[2 * g];
            o[HD + 1] = sml[2 * g + 1];
        }
    }
}

// Register-resident split-KV attention, used when G = hq / hkv <= 8 (GP = G
// rounded up to a power of two).  Same grid, tile and partial layout as k_attn;
// no LDS round trip for K and V:
//   * wave w owns positions t0 + 16w .. t0 + 16w + 15; lane (c, rg) holds float4
//     column c of K and V for its NI positions i * RPL + rg (every load in
//     flight at once) and column c of the G query heads;
//   * per lane 4-element partial dots for all (position, head) pairs, then one
//     transpose reduction over the C4 lanes of a row leaves each (position,
//     head) score in exactly one representative lane;
//   * per wave and head: max m and l = sum e^(s - m) by butterflies over the
//     lane bits that do not encode the head; the probabilities go through a
//     2 KB LDS table to the lanes holding V, which accumulate o per head and
//     fold their row groups with two shuffles;
//   * the four waves' (o, m, l) combine through LDS into the block's partial.
// Block y folds tiles y, y + gridDim.y, ... below the sequence length into one
// running (o, m, l) per (head, column) -- the online softmax across tiles --
// and writes it as partial y; with one tile per block that is the tile's own.
template <int HD, int GP>
__global__ __launch_bounds__(256) void k_attn_reg(const DecState *__restrict__ st,
                                                  const float *__restrict__ qkv,
                                                  const float *__restrict__ kc,
                                                  const float *__restrict__ vc,
                                                  float *__restrict__ part, int G, int max_seq,
                                                  int nsplit, float scale, int cap) {
    constexpr int T = kAttnTile;
    constexpr int PW = T / 4;              // positions per wave
    constexpr int C4 = HD / 4;             // lanes per position row
    constexpr int B = Log2<C4>::value;
    constexpr int RPL = 64 / C4;           // positions per wave-wide load
    constexpr int NI = PW / RPL;           // positions per lane
    constexpr int NV = NI * GP;            // (position, head) partials per lane
    constexpr int CH = NV < C4 ? NV : C4;  // partials reduced per transpose pass
    constexpr int NCH = NV / CH;
    constexpr int LGP = Log2<GP>::value;
    constexpr int RB = B - Log2<CH>::value;   // low lane bits that hold replicas
    static_assert(T == 64 && PW % RPL == 0 && GP <= C4, "attention tile layout");
    __shared__ float sp[4][PW][GP];
    __shared__ float so[4][GP][HD];
    __shared__ float sml[4][GP][2];

    const int kvh = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int c = lane & (C4 - 1), rg = lane >> B;
    // column c of the G query heads: the same for every tile, and loaded
    // before the step position is known
    const float4 *q4 = reinterpret_cast<const float4 *>(qkv) + (size_t)kvh * G * C4 + c;
    float4 qr[GP];
#pragma unroll
    for (int g = 0; g < GP; ++g)
        qr[g] = g < G ? q4[(size_t)g * C4] : make_float4(0.f, 0.f, 0.f, 0.f);
    const int seq = min(st->pos + 1, cap);
    if ((int)blockIdx.y * T >= seq) return;   // no tile: the merge never reads this partial
    // the running (o, m, l) of this thread's (head, column) of the final fold
    // (G * C4 <= 256: one per thread at most)
    float4 run_o = make_float4(0.f, 0.f, 0.f, 0.f);
    float run_m = -FLT_MAX, run_l = 0.f;
    for (int spl = blockIdx.y; spl * T < seq; spl += gridDim.y) {
        const int t0 = spl * T;
        const int pbase = t0 + wave * PW;

        const float4 *k4 = reinterpret_cast<const float4 *>(kc) + (size_t)kvh * max_seq * C4 + c;
        const float4 *v4 = reinterpret_cast<const float4 *>(vc) + (size_t)kvh * max_seq * C4 + c;
        float4 kr[NI], vr[NI];
        // every K row, then every V row: the scores and the softmax wait only
        // for K, and run while V is still arriving.
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int p = pbase + i * RPL + rg;
            kr[i] = p < seq ? load_nt_f4(reinterpret_cast<const float *>(k4 + (size_t)p * C4))
                            : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int p = pbase + i * RPL + rg;
            vr[i] = p < seq ? load_nt_f4(reinterpret_cast<const float *>(v4 + (size_t)p * C4))
                            : make_float4(0.f, 0.f, 0.f, 0.f);
        }

        float v[NV];
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int g = 0; g < GP; ++g)
                v[i * GP + g] =
                    fmaf(qr[g].w, kr[i].w,
                         fmaf(qr[g].z, kr[i].z, fmaf(qr[g].y, kr[i].y, qr[g].x * kr[i].x)));

        // Lane l now holds, per chunk ch, the score of flat index ch * CH + (c >> RB).
        const int vi = c >> RB;
        const int g = vi & (GP - 1);
        const bool rep = (c & ((1 << RB) - 1)) == 0;
        float sc[NCH];
        bool ok[NCH];
        int pw[NCH];
        float m = -FLT_MAX;
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
            float t[CH];
#pragma unroll
            for (int j = 0; j < CH; ++j) t[j] = v[ch * CH + j];
            transpose_reduce<CH>(t, lane, B);
            const int i = (ch * CH + vi) >> LGP;
            pw[ch] = i * RPL + rg;
            ok[ch] = g < G && pbase + pw[ch] < seq;
            sc[ch] = t[0] * scale;
            if (ok[ch]) m = fmaxf(m, sc[ch]);
        }
#pragma unroll
        for (int j = 0; j < 6; ++j)
            if (j < RB || j >= RB + LGP) m = fmaxf(m, shfl_xor_u(m, 1 << j));
        float l = 0.f;
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
            const float p = ok[ch] ? expf(sc[ch] - m) : 0.f;
            if (rep) sp[wave][pw[ch]][g] = p;
            if (rep) l += p;
        }
#pragma unroll
        for (int j = 0; j < 6; ++j)
            if (j < RB || j >= RB + LGP) l += shfl_xor_u(l, 1 << j);
        if (rg == 0 && rep && vi < GP) {
            sml[wave][g][0] = m;
            sml[wave][g][1] = l;
        }
        __syncthreads();

        float4 acc[GP];
#pragma unroll
        for (int h = 0; h < GP; ++h) acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const float *pr = sp[wave][i * RPL + rg];
#pragma unroll
            for (int h = 0; h < GP; ++h) {
                const float p = pr[h];
                acc[h].x = fmaf(p, vr[i].x, acc[h].x);
                acc[h].y = fmaf(p, vr[i].y, acc[h].y);
                acc[h].z = fmaf(p, vr[i].z, acc[h].z);
                acc[h].w = fmaf(p, vr[i].w, acc[h].w);
            }
        }
#pragma unroll
        for (int j = B; j < 6; ++j)
#pragma unroll
            for (int h = 0; h < GP; ++h) {
                acc[h].x += shfl_xor_u(acc[h].x, 1 << j);
                acc[h].y += shfl_xor_u(acc[h].y, 1 << j);
                acc[h].z += shfl_xor_u(acc[h].z, 1 << j);
                acc[h].w += shfl_xor_u(acc[h].w, 1 << j);
            }
        if (rg == 0) {
#pragma unroll
            for (int h = 0; h < GP; ++h)
                if (h < G) *reinterpret_cast<float4 *>(&so[wave][h][4 * c]) = acc[h];
        }
        __syncthreads();

        if (tid < G * C4) {
            const int h = tid / C4, cc = tid - h * C4;
            float M = -FLT_MAX;
#pragma unroll
            for (int w = 0; w < 4; ++w) M = fmaxf(M, sml[w][h][0]);
            float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
            float L = 0.f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float e = expf(sml[w][h][0] - M);
                const float4 ow = *reinterpret_cast<const float4 *>(&so[w][h][4 * cc]);
                o.x = fmaf(e, ow.x, o.x);
                o.y = fmaf(e, ow.y, o.y);
                o.z = fmaf(e, ow.z, o.z);
                o.w = fmaf(e, ow.w, o.w);
                L = fmaf(e, sml[w][h][1], L);
            }
            // fold the tile into the running state (first tile: a = 0, b = 1,
            // so a single tile passes through unchanged)
            const float mn = fmaxf(run_m, M);
            const float a = expf(run_m - mn), b = expf(M - mn);
            run_o = make_float4(fmaf(run_o.x, a, o.x * b), fmaf(run_o.y, a, o.y * b),
                                fmaf(run_o.z, a, o.z * b), fmaf(run_o.w, a, o.w * b));
            run_l = fmaf(run_l, a, L * b);
            run_m = mn;
        }
        __syncthreads();   // the next tile rewrites sp, so and sml
    }
    if (tid < G * C4) {
        const int h = tid / C4, cc = tid - h * C4;
        float *dst = part + ((size_t)(kvh * G + h) * nsplit + blockIdx.y) * (HD + 4);
        *reinterpret_cast<float4 *>(dst + 4 * cc) = run_o;
        if (cc == 0) {
            dst[HD] = run_m;
            dst[HD + 1] = run_l;
        }
    }
}

// Merge of one query head's tiles: M = max m_s, L = sum e^(m_s - M) l_s,
// o = sum e^(m_s - M) o_s / L; then the head's x chunk records for the O
// projection.  blockDim = 64: thread = (half of the tiles, float4 column).
template <int HD>
__global__ __launch_bounds__(64) void k_attn_merge(const DecState *__restrict__ st,
                                                   const float *__restrict__ part,
                                                   float *__restrict__ out,
                                                   uint32_t *__restrict__ xq, int nsplit,
                                                   int cap) {
    constexpr int C4 = HD / 4;
    constexpr size_t rec = HD + 4;
    __shared__ float sw[kMaxTiles];
    __shared__ float sacc[2 * HD];
    __shared__ float so[HD];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int used = (min(st->pos + 1, cap) + kAttnTile - 1) / kAttnTile;
    const float *ph = part + (size_t)h * nsplit * rec;
    float M = -FLT_MAX;
    for (int s = tid; s < used; s += 64) M = fmaxf(M, ph[s * rec + HD]);
    M = wave_max(M);
    float L = 0.f;
    for (int s = tid; s < used; s += 64) {
        const float w = expf(ph[s * rec + HD] - M);
        sw[s] = w;
        L = fmaf(w, ph[s * rec + HD + 1], L);
    }
    L = wave_sum(L);
    __syncthreads();
    if (tid < 2 * C4) {
        const int half = tid / C4, c = tid - half * C4;
        const float *pc = ph + 4 * c;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int s0 = half; s0 < used; s0 += 32) {
            float4 v[16];
            float w[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int s = s0 + 2 * u;
                const bool ok = s < used;
                v[u] = ok ? *reinterpret_cast<const float4 *>(pc + s * rec)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
                w[u] = ok ? sw[s] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                acc.x = fmaf(w[u], v[u].x, acc.x);
                acc.y = fmaf(w[u], v[u].y, acc.y);
                acc.z = fmaf(w[u], v[u].z, acc.z);
                acc.w = fmaf(w[u], v[u].w, acc.w);
            }
        }
        *reinterpret_cast<float4 *>(sacc + half * HD + 4 * c) = acc;
    }
    __syncthreads();
    const float inv = 1.0f / fmaxf(L, 1e-30f);
    for (int d = tid; d < HD; d += 64) {
        const float v = (sacc[d] + sacc[HD + d]) * inv;
        so[d] = v;
        out[(size_t)h * HD + d] = v;
    }
    __syncthreads();
    if (xq) {
        constexpr int NREC = HD / 32;   // records of this head: 8 lanes each
        const int rc = tid >> 3, sub = tid & 7;
        const bool live = rc < NREC;
        const float4 vv = live ? reinterpret_cast<const float4 *>(so + rc * 32)[sub]
                               : make_float4(0.f, 0.f, 0.f, 0.f);
        build_xrec8(vv, sub, live, xq, (int)gridDim.x * NREC, h * NREC + (live ? rc : 0));
    }
}

// Merge of one 32-column chunk of one query head's tiles: grid (hq, HD / 32),
// 64 threads = 8 split groups x 8 float4 columns.  Thread (sg, c) folds the
// (o, m, l) of splits sg, sg + 8, ... with all of a pass's loads in flight;
// the groups combine through LDS: M = max m_s, L = sum e^(m_s - M) l_s,
// o = sum e^(m_s - M) o_s / max(L, 1e-30) (src/llm/decoder.rs:1148-1213).
// Lanes 0..7 then hold the chunk and write o and its x chunk record.
template <int HD>
__global__ __launch_bounds__(64) void k_attn_merge_chunk(const DecState *__restrict__ st,
                                                         const float *__restrict__ part,
                                                         float *__restrict__ out,
                                                         uint32_t *__restrict__ xq, int nsplit,
                                                         int cap) {
    constexpr int NSG = 8, NB = 12;
    constexpr size_t rec = HD + 4;
    __shared__ float4 so4[NSG][8];
    __shared__ float smx[NSG], sl[NSG];
    const int h = blockIdx.x, ck = blockIdx.y, tid = threadIdx.x;
    const int c = tid & 7, sg = tid >> 3;
    // partials written: one per attention block that had a tile
    const int used = min(nsplit, (min(st->pos + 1, cap) + kAttnTile - 1) / kAttnTile);
    const float *ph = part + (size_t)h * nsplit * rec;
    float M = -FLT_MAX, L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    // The passes cover all nsplit slots of the buffer: a pass's loads do not
    // wait for the step position, which only masks the slots not written
    // this step afterwards.
    for (int s0 = 0; s0 < nsplit; s0 += NSG * NB) {
        float4 ov[NB];
        float mv[NB], lv[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int sp = s0 + sg + u * NSG;
            const float *pp = ph + (size_t)(sp < nsplit ? sp : 0) * rec;
            const float4 o4 = *reinterpret_cast<const float4 *>(pp + 32 * ck + 4 * c);
            const float m4 = pp[HD], l4 = pp[HD + 1];
            const bool ok = sp < used;
            ov[u] = ok ? o4 : make_float4(0.f, 0.f, 0.f, 0.f);
            mv[u] = ok ? m4 : -FLT_MAX;
            lv[u] = ok ? l4 : 0.f;
        }
        float mn = M;
#pragma unroll
        for (int u = 0; u < NB; ++u) mn = fmaxf(mn, mv[u]);
        const float a = expf(M - mn);
        acc = make_float4(acc.x * a, acc.y * a, acc.z * a, acc.w * a);
        L *= a;
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const float w = expf(mv[u] - mn);
            acc.x = fmaf(w, ov[u].x, acc.x);
            acc.y = fmaf(w, ov[u].y, acc.y);
            acc.z = fmaf(w, ov[u].z, acc.z);
            acc.w = fmaf(w, ov[u].w, acc.w);
            L = fmaf(w, lv[u], L);
        }
        M = mn;
    }
    so4[sg][c] = acc;
    if (c == 0) {
        smx[sg] = M;
        sl[sg] = L;
    }
    __syncthreads();
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    if (tid < 8) {
        float mg = -FLT_MAX;
#pragma unroll
        for (int g = 0; g < NSG; ++g) mg = fmaxf(mg, smx[g]);
        float lt = 0.f;
#pragma unroll
        for (int g = 0; g < NSG; ++g) {
            const float w = expf(smx[g] - mg);
            const float4 v = so4[g][tid];
            o.x = fmaf(w, v.x, o.x);
            o.y = fmaf(w, v.y, o.y);
            o.z = fmaf(w, v.z, o.z);
            o.w = fmaf(w, v.w, o.w);
            lt = fmaf(w, sl[g], lt);
        }
        const float inv = 1.0f / fmaxf(lt, 1e-30f);
        o = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
        reinterpret_cast<float4 *>(out + (size_t)h * HD + 32 * ck)[tid] = o;
    }
    // the whole wave takes part (8-lane groups); lanes 0..7 hold the chunk
    if (xq) build_xrec8(o, tid & 7, tid < 8, xq, (int)(gridDim.x * gridDim.y), h * (HD / 32) + ck);
}

// Greedy argmax, stage 1: per block the largest logit, lowest index on ties
// (the reference's strict `>` scan, src/llm/decoder.rs:914-925).  NaN at index 0
// wins outright (the scan never replaces a NaN best); NaN elsewhere never wins.
__device__ __forceinline__ void better(float &bv, int &bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

__global__ __launch_bounds__(256) void k_argmax_partial(const float *__restrict__ logits, int n,
                                                        float *__restrict__ pv,
                                                        int *__restrict__ pi) {
    __shared__ float sv[256];
    __shared__ int si[256];
    float bv = -INFINITY;
    int bi = INT_MAX;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        float v = logits[i];
        if (__builtin_isnan(v)) v = (i == 0) ? INFINITY : -INFINITY;
        better(bv, bi, v, i);
    }
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int s = blockDim.x / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) {
            float v = sv[threadIdx.x + s];
            int i = si[threadIdx.x + s];
            float b = sv[threadIdx.x];
            int j = si[threadIdx.x];
            better(b, j, v, i);
            sv[threadIdx.x] = b;
            si[threadIdx.x] = j;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = sv[0];
        pi[blockIdx.x] = si[0];
    }
}

// Stage 2: final argmax, then the greedy loop's state update on the device:
// history[step] = token; token = argmax; pos += 1; step += 1.
__global__ __launch_bounds__(256) void k_argmax_final(const float *__restrict__ pv,
                                                      const int *__restrict__ pi, int nb, int n,
                                                      DecState *__restrict__ st,
                                                      int *__restrict__ history, int hist_cap) {
    __shared__ float sv[256];
    __shared__ int si[256];
    float bv = -INFINITY;
    int bi = INT_MAX;
    for (int i = threadIdx.x; i < nb; i += blockDim.x) better(bv, bi, pv[i], pi[i]);
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int s = blockDim.x / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) {
            float b = sv[threadIdx.x];
            int j = si[threadIdx.x];
            better(b, j, sv[threadIdx.x + s], si[threadIdx.x + s]);
            sv[threadIdx.x] = b;
            si[threadIdx.x] = j;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        int tok = si[0];
        if (tok < 0 || tok >= n) tok = 0;
        const int step = st->step;
        if (history && step < hist_cap) history[step] = tok;
        st->argmax = tok;
        st->token = tok;
        st->pos = st->pos + 1;
        st->step = step + 1;
    }
}


// ---------------------------------------------------------------------------
// Batched prefill (M consecutive prompt positions per launch)
// ---------------------------------------------------------------------------

// X[m] = embed[tok[m]] (tokens validated on the host).
__global__ __launch_bounds__(256) void k_embed_rows(const int *__restrict__ tok,
                                                    const float *__restrict__ embed,
                                                    float *__restrict__ X, int H) {
    const float4 *src = reinterpret_cast<const float4 *>(embed + (size_t)tok[blockIdx.x] * H);
    float4 *dst = reinterpret_cast<float4 *>(X + (size_t)blockIdx.x * H);
    for (int i = threadIdx.x; i < H / 4; i += blockDim.x) dst[i] = src[i];
}

// RMSNorm of one row per block, with k_rmsnorm's arithmetic (the same
// per-thread sum order and two roundings of (x * inv) * w).
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const float *__restrict__ X,
                                                      const float *__restrict__ w,
                                                      float *__restrict__ Xn, int H, float eps) {
    __shared__ float scratch[16];
    const int tid = threadIdx.x;
    const float4 *s4 = reinterpret_cast<const float4 *>(X + (size_t)blockIdx.x * H);
    float ss = 0.f;
    for (int i = tid; i < H / 4; i += blockDim.x) {
        const float4 v = s4[i];
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
    }
    const float tot = block_sum(ss, scratch);
    const float inv = 1.0f / sqrtf(tot / (float)H + eps);
    float4 *d4 = reinterpret_cast<float4 *>(Xn + (size_t)blockIdx.x * H);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    for (int i = tid; i < H / 4; i += blockDim.x) {
        const float4 v = s4[i], ww = w4[i];
        d4[i] = make_float4(__fmul_rn(__fmul_rn(v.x, inv), ww.x), __fmul_rn(__fmul_rn(v.y, inv), ww.y),
                            __fmul_rn(__fmul_rn(v.z, inv), ww.z), __fmul_rn(__fmul_rn(v.w, inv), ww.w));
    }
}

// RoPE of the q and k heads of row m (position start + m) and the KV-cache
// append, as the decode epilogue does it (decoder.rs:28-68, 1137-1146):
// q1' = q1 c[i] - q2 s[i], q2' = q2 c[i + d/2] + q1 s[i + d/2], products
// rounded separately.  Grid (M, hq + 2 hkv), hd / 2 threads.
__global__ void k_rope_rows(const float *__restrict__ qkv, int nq, float *__restrict__ q,
                            float *__restrict__ kc, float *__restrict__ vc,
                            const float *__restrict__ cos_t, const float *__restrict__ sin_t,
                            int start, int hq, int hkv, int hd, int max_seq) {
    const int m = blockIdx.x, head = blockIdx.y, i = threadIdx.x, half = hd >> 1;
    const int pos = start + m;
    const float *src = qkv + (size_t)m * nq + (size_t)head * hd;
    const float x1 = src[i], x2 = src[i + half];
    if (head < hq + hkv) {
        const float *cr = cos_t + (size_t)pos * hd, *sr = sin_t + (size_t)pos * hd;
        const float y1 = __fsub_rn(__fmul_rn(x1, cr[i]), __fmul_rn(x2, sr[i]));
        const float y2 = __fadd_rn(__fmul_rn(x2, cr[i + half]), __fmul_rn(x1, sr[i + half]));
        float *dst = head < hq ? q + ((size_t)m * hq + head) * hd
                               : kc + ((size_t)(head - hq) * max_seq + pos) * hd;
        dst[i] = y1;
        dst[i + half] = y2;
    } else {
        float *dst = vc + ((size_t)(head - hq - hkv) * max_seq + pos) * hd;
        dst[i] = x1;
        dst[i + half] = x2;
    }
}

// Causal GQA attention of M consecutive query positions start .. start+M-1
// over the cache (query at position p sees keys 0..p; decoder.rs:1148-1213),
// on FP32 MFMA (v_mfma_f32_16x16x4f32).  out [M][hq * HD].
//
// A block owns one KV head and a tile of query rows, where the rows of a KV
// head are its (position m, head g of the group) pairs, i = m * G + g: every
// query head that shares the KV head reads each K / V tile from the same LDS
// copy, and a short verify chunk (M * G rows) fills one small tile instead of
// padding a position tile per head.  K and V tiles of KT positions are staged
// in LDS (zero past the last position the tile needs); online softmax with a
// running max and sum per row, then 1 / max(sum, 1e-30).
//
// Key-range split (blockIdx.z of nsplit, tps tiles each): with nsplit > 1 the
// block writes its unnormalised o, running max and sum to part / pml and
// k_prefill_merge combines the splits, so few query rows over a long cache
// (verify_tokens, short chunks after a long prefix) still fill the chip.
//
// Query tiles of 64 / KG rows.  The four waves take the tile's 16-row blocks
// and, with KG > 1 (few rows: verify_tokens, short chunks), KG groups of each
// key tile's positions: wave w takes row block w % (4 / KG) and key group
// w / (4 / KG), keeps its own online softmax over the key tiles of its split,
// and the key groups' (o, m, l) meet in LDS at the end.  MFMA operands: lane
// (g, c) = (lane / 16, lane % 16) supplies A[c][g] and B[g][c], and gets
// D[4g + r][c] in register r; lane group g takes the contiguous quarter
// g * (K / 4) .. of each contraction, so its operands are 16-byte LDS reads.
// Per tile and wave:
//   S (16 x KT / KG) = Q K^T: A = the wave's q rows (registers, from the
//     start), B = its keys (LDS, every read issued before the MFMAs, the key
//     blocks' chains interleaved);
//   causal mask, scale and the online softmax in the MFMA result layout
//     (lane (g, c) holds rows 4g..4g+3 at key c of every 16-key block): row
//     max and sum by DPP butterflies over the 16 lanes of a row group, and
//     each row's rescale of o lands in the lane's own registers;
//   P goes through the wave's own LDS rows from the result to the A layout;
//   O (16 x HD) += P V: A = P, B = its values (LDS, read ahead of the MFMAs,
//     one chain per 16 output columns).
// The next tile's K / V loads are in flight during the MFMAs.  A wave whose
// rows are all padding only helps load the tiles.
template <int HD, int KT, int KG>
__global__ __launch_bounds__(256) void k_prefill_attn_mfma(const float *__restrict__ q,
                                                           const float *__restrict__ kc,
                                                           const float *__restrict__ vc,
                                                           float *__restrict__ out, int start,
                                                           int M, int hq, int hkv, int max_seq,
                                                           float scale, int tps,
                                                           float *__restrict__ part,
                                                           float *__restrict__ pml) {
    typedef float f32x4_t __attribute__((ext_vector_type(4)));
    constexpr int RB = 4 / KG;             // row blocks of 16 per tile
    constexpr int QT = 16 * RB, KW = KT / KG;   // query rows per tile, keys per wave per tile
    constexpr int KP = HD + 4, NB = KW / 16, NS = HD / 4, OB = HD / 16, C4 = HD / 4;
    constexpr int KS = KW / 4;   // keys per lane group in the P V contraction
    static_assert(KW >= 16, "a wave takes whole 16-key blocks");
    __shared__ __attribute__((aligned(16))) float sk[KT > QT ? KT : QT][KP];
    __shared__ __attribute__((aligned(16))) float sv[KT][KP];
    __shared__ __attribute__((aligned(16))) float sp[4][16][KW + 4];
    const int G = hq / hkv, NR = M * G;
    const int kvh = blockIdx.y, i0 = blockIdx.x * QT;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, g = lane >> 4, c = lane & 15;
    const int rb = wave % RB, kg = wave / RB;   // row block, key group
    const int w0 = i0 + 16 * rb;   // first row of this wave
    const bool busy = w0 < NR;       // wave-uniform
    const int last = start + (min(i0 + QT, NR) - 1) / G;   // last position any row sees
    const int ntiles = last / KT + 1;
    const int kt0 = blockIdx.z * tps, kt1 = min(ntiles, kt0 + tps);
    const float *kb = kc + (size_t)kvh * max_seq * HD, *vb = vc + (size_t)kvh * max_seq * HD;
    // A tile's K and V rows go global -> registers -> LDS; the next tile's
    // loads are in flight while the current one is multiplied (rows past
    // `last` read row `last` and are stored as zeros).
    constexpr int NL = KT * C4 / 256;
    float4 kv[NL], vv[NL];
    auto load_tile = [&](int kt) {
#pragma unroll
        for (int u = 0; u < NL; ++u) {
            const int i = t + 256 * u, j = i / C4, c4 = i - j * C4;
            const int p = min(kt * KT + j, last);
            kv[u] = reinterpret_cast<const float4 *>(kb + (size_t)p * HD)[c4];
        }
#pragma unroll
        for (int u = 0; u < NL; ++u) {
            const int i = t + 256 * u, j = i / C4, c4 = i - j * C4;
            const int p = min(kt * KT + j, last);
            vv[u] = reinterpret_cast<const float4 *>(vb + (size_t)p * HD)[c4];
        }
    };
    // the tile's q rows through LDS into the A-operand registers, loaded
    // together with the first K / V tile
    {
        constexpr int NQ = QT * C4 / 256;
        float4 v[NQ];
#pragma unroll
        for (int u = 0; u < NQ; ++u) {
            const int i = t + 256 * u, r = i / C4, c4 = i - r * C4, ii = i0 + r;
            const int iq = ii < NR ? ii : 0;
            const int m = iq / G, h = kvh * G + (iq - m * G);
            v[u] = reinterpret_cast<const float4 *>(q + ((size_t)m * hq + h) * HD)[c4];
            if (ii >= NR) v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (kt0 < kt1) load_tile(kt0);
#pragma unroll
        for (int u = 0; u < NQ; ++u) {
            const int i = t + 256 * u, r = i / C4, c4 = i - r * C4;
            *reinterpret_cast<float4 *>(&sk[r][4 * c4]) = v[u];
        }
    }
    __syncthreads();
    float qa[NS];   // q[row w0 + c][g * NS + s]
#pragma unroll
    for (int s = 0; s < NS; s += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(&sk[16 * rb + c][g * NS + s]);
        qa[s] = v.x; qa[s + 1] = v.y; qa[s + 2] = v.z; qa[s + 3] = v.w;
    }
    float mrun[4], lrun[4];
    int pq[4];
    f32x4_t o[OB];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        mrun[r] = -INFINITY;
        lrun[r] = 0.f;
        pq[r] = start + (w0 + 4 * g + r) / G;   // past `last` for padding rows: finite scores
    }
#pragma unroll
    for (int b = 0; b < OB; ++b) o[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int kt = kt0; kt < kt1; ++kt) {
        __syncthreads();   // every wave is done with sk / sv (and the q rows)
#pragma unroll
        for (int u = 0; u < NL; ++u) {
            const int i = t + 256 * u, j = i / C4, c4 = i - j * C4;
            const bool in = kt * KT + j <= last;
            *reinterpret_cast<float4 *>(&sk[j][4 * c4]) =
                in ? kv[u] : make_float4(0.f, 0.f, 0.f, 0.f);
            *reinterpret_cast<float4 *>(&sv[j][4 * c4]) =
                in ? vv[u] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        __syncthreads();
        if (kt + 1 < kt1) load_tile(kt + 1);
        if (!busy) continue;
        // S = Q K^T over the wave's keys kg * KW .. of the tile: the keys
        // first, then the MFMAs
        float kr[NB][NS];   // k[key kg * KW + 16 b + c][g * NS + s]
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int s = 0; s < NS; s += 4) {
                const float4 v =
                    *reinterpret_cast<const float4 *>(&sk[kg * KW + 16 * b + c][g * NS + s]);
                kr[b][s] = v.x; kr[b][s + 1] = v.y; kr[b][s + 2] = v.z; kr[b][s + 3] = v.w;
            }
        __builtin_amdgcn_sched_barrier(0);
        f32x4_t sacc[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) sacc[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int b = 0; b < NB; ++b)
                sacc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[s], kr[b][s], sacc[b], 0, 0, 0);
        // sacc[b][r] = S[row 4 g + r][key kg * KW + 16 b + c]
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float sc[NB];
            float mt = -INFINITY;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int pk = kt * KT + kg * KW + 16 * b + c;
                sc[b] = pk <= pq[r] ? sacc[b][r] * scale : -INFINITY;
                mt = fmaxf(mt, sc[b]);
            }
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) mt = fmaxf(mt, shfl_xor_u(mt, off));
            const float mn = fmaxf(mrun[r], mt);
            // all-masked so far: nothing to rescale, every p is 0
            const float alpha = mn == -INFINITY ? 1.f : expf(mrun[r] - mn);
            float ls = 0.f;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const float pj = mn == -INFINITY ? 0.f : expf(sc[b] - mn);
                sp[wave][4 * g + r][16 * b + c] = pj;
                ls += pj;
            }
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) ls += shfl_xor_u(ls, off);
            lrun[r] = lrun[r] * alpha + ls;
            mrun[r] = mn;
#pragma unroll
            for (int b = 0; b < OB; ++b) o[b][r] *= alpha;
        }
        // the wave's P rows: written above by their owners, read below across lanes
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // O += P V: P[row c][key g * KS + s] and V[key kg * KW + g * KS + s][col 16 b + c]
        float pa[KS];
#pragma unroll
        for (int s = 0; s < KS; s += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(&sp[wave][c][g * KS + s]);
            pa[s] = v.x; pa[s + 1] = v.y; pa[s + 2] = v.z; pa[s + 3] = v.w;
        }
        constexpr int OG = OB < 4 ? OB : 4;   // output column blocks per batch of reads
#pragma unroll
        for (int b0 = 0; b0 < OB; b0 += OG) {
            float vr[OG][KS];
#pragma unroll
            for (int bb = 0; bb < OG; ++bb)
#pragma unroll
                for (int s = 0; s < KS; ++s)
                    vr[bb][s] = sv[kg * KW + g * KS + s][16 * (b0 + bb) + c];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < KS; ++s)
#pragma unroll
                for (int bb = 0; bb < OG; ++bb)
                    o[b0 + bb] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[s], vr[bb][s],
                                                                      o[b0 + bb], 0, 0, 0);
        }
        // the next tile's P writes wait for these reads
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (KG > 1) {
        // key groups 1.. hand their (o, m, l) to group 0 through LDS (sk)
        __syncthreads();
        float *xo = &sk[0][0];                          // [KG - 1][RB][16][HD]
        float *xm = xo + (KG - 1) * RB * 16 * HD;       // [KG - 1][RB][16][2]
        if (kg > 0 && busy) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float *row = xo + (((kg - 1) * RB + rb) * 16 + 4 * g + r) * HD;
#pragma unroll
                for (int b = 0; b < OB; ++b) row[16 * b + c] = o[b][r];
                if (c == 0) {
                    float *ml = xm + (((kg - 1) * RB + rb) * 16 + 4 * g + r) * 2;
                    ml[0] = mrun[r];
                    ml[1] = lrun[r];
                }
            }
        }
        __syncthreads();
        if (kg > 0) return;
        if (busy) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float mg = mrun[r];
#pragma unroll
                for (int j = 1; j < KG; ++j)
                    mg = fmaxf(mg, xm[(((j - 1) * RB + rb) * 16 + 4 * g + r) * 2]);
                // every group all-masked: keep o = 0, l = 0 (m = -inf)
                const float a0 = mg == -INFINITY ? 1.f : expf(mrun[r] - mg);
                float l = lrun[r] * a0;
#pragma unroll
                for (int b = 0; b < OB; ++b) o[b][r] *= a0;
#pragma unroll
                for (int j = 1; j < KG; ++j) {
                    const int slot = ((j - 1) * RB + rb) * 16 + 4 * g + r;
                    const float mj = xm[slot * 2];
                    const float aj = mg == -INFINITY ? 0.f : expf(mj - mg);
                    l = fmaf(xm[slot * 2 + 1], aj, l);
#pragma unroll
                    for (int b = 0; b < OB; ++b) o[b][r] = fmaf(xo[slot * HD + 16 * b + c], aj, o[b][r]);
                }
                mrun[r] = mg;
                lrun[r] = l;
            }
        }
    }
    if (!busy) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int ii = w0 + 4 * g + r;
        if (ii >= NR) continue;
        const int m = ii / G, h = kvh * G + (ii - m * G);
        if (part) {   // one split of several: unnormalised o, max and sum
            const size_t row = ((size_t)blockIdx.z * M + m) * hq + h;
#pragma unroll
            for (int b = 0; b < OB; ++b) part[row * HD + 16 * b + c] = o[b][r];
            if (c == 0) {
                pml[row * 2] = mrun[r];
                pml[row * 2 + 1] = lrun[r];
            }
        } else {
            const float inv = 1.0f / fmaxf(lrun[r], 1e-30f);
#pragma unroll
            for (int b = 0; b < OB; ++b) out[((size_t)m * hq + h) * HD + 16 * b + c] = o[b][r] * inv;
        }
    }
}

// Combines the key-range splits of one (row, head): M = max m_s,
// l = sum l_s e^(m_s - M), o = sum o_s e^(m_s - M) / max(l, 1e-30).  Splits
// past a row's last tile hold m = -inf and contribute nothing.  256 threads =
// SG split groups x HD / 4 float4 columns; each thread folds splits sg, sg +
// SG, ... NB at a time (all NB loads in flight) with its own running max, and
// the split groups combine through LDS.
template <int HD>
__global__ __launch_bounds__(256) void k_prefill_merge(const float *__restrict__ part,
                                                      const float *__restrict__ pml,
                                                      float *__restrict__ out, int M, int hq,
                                                      int nsplit) {
    constexpr int C4 = HD / 4, SG = 256 / C4, NB = 8;
    __shared__ float4 so[SG][C4];
    __shared__ float smx[SG], sl[SG];
    const int m = blockIdx.x, h = blockIdx.y, c = threadIdx.x % C4, sg = threadIdx.x / C4;
    float mx = -INFINITY, l = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = sg; s0 < nsplit; s0 += SG * NB) {
        float ms[NB], ls[NB];
        float4 ov[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int sp = s0 + u * SG;
            const bool ok = sp < nsplit;
            const size_t row = ((size_t)(ok ? sp : 0) * M + m) * hq + h;
            ms[u] = ok ? pml[row * 2] : -INFINITY;
            ls[u] = ok ? pml[row * 2 + 1] : 0.f;
            ov[u] = ok ? reinterpret_cast<const float4 *>(part + row * HD)[c]
                       : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        float mn = mx;
#pragma unroll
        for (int u = 0; u < NB; ++u) mn = fmaxf(mn, ms[u]);
        if (mn == -INFINITY) continue;   // nothing seen yet
        const float a = mx == -INFINITY ? 0.f : expf(mx - mn);
        acc = make_float4(acc.x * a, acc.y * a, acc.z * a, acc.w * a);
        l *= a;
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const float w = ms[u] == -INFINITY ? 0.f : expf(ms[u] - mn);
            l = fmaf(ls[u], w, l);
            acc.x = fmaf(ov[u].x, w, acc.x);
            acc.y = fmaf(ov[u].y, w, acc.y);
            acc.z = fmaf(ov[u].z, w, acc.z);
            acc.w = fmaf(ov[u].w, w, acc.w);
        }
        mx = mn;
    }
    so[sg][c] = acc;
    if (c == 0) {
        smx[sg] = mx;
        sl[sg] = l;
    }
    __syncthreads();
    if (sg == 0) {
        float mg = -INFINITY;
#pragma unroll
        for (int g = 0; g < SG; ++g) mg = fmaxf(mg, smx[g]);
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        float lt = 0.f;
#pragma unroll
        for (int g = 0; g < SG; ++g) {
            const float w = smx[g] == -INFINITY ? 0.f : expf(smx[g] - mg);
            const float4 v = so[g][c];
            o.x = fmaf(v.x, w, o.x);
            o.y = fmaf(v.y, w, o.y);
            o.z = fmaf(v.z, w, o.z);
            o.w = fmaf(v.w, w, o.w);
            lt = fmaf(sl[g], w, lt);
        }
        const float inv = 1.0f / fmaxf(lt, 1e-30f);
        reinterpret_cast<float4 *>(out + ((size_t)m * hq + h) * HD)[c] =
            make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
    }
}

}  // namespace

int launch_rmsnorm(const DecState *st, const float *embed, float *x, const float *w, float *xn,
                   uint32_t *xq, int H, float eps, hipStream_t s) {
    TB_REQUIRE(H <= kMaxHidden && H % 32 == 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: hidden size must be a multiple of 32 and <= " +
                   std::to_string(kMaxHidden));
    const int blocks = (H / 32 + kNormChunks - 1) / kNormChunks;
    hipLaunchKernelGGL(k_rmsnorm, dim3(blocks), dim3(256), 0, s, st, embed, x, w, xn, xq, H, eps);
    TB_LAUNCHED();
    return TB_OK;
}

int launch_embed_rec(const DecState *st, const float *embed, float *x, const float *w,
                     float *xw, uint32_t *xq, float *ssq, int H, hipStream_t s) {
    TB_REQUIRE(H % 32 == 0, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: hidden size must be a multiple of 32");
    const int threads = H / 4;
    hipLaunchKernelGGL(k_embed_rec, dim3((threads + 255) / 256), dim3(256), 0, s, st, embed, x, w,
                       xw, xq, ssq, H);
    TB_LAUNCHED();
    return TB_OK;
}

int launch_rope_kv(const DecState *st, float *qkv, const float *cos_t, const float *sin_t,
                   float *kc, float *vc, int hq, int hkv, int hd, int max_seq, hipStream_t s) {
    hipLaunchKernelGGL(k_rope_kv, dim3(hq + 2 * hkv), dim3(hd / 2), 0, s, st, qkv, cos_t, sin_t,
                       kc, vc, hq, hkv, hd, max_seq);
    TB_LAUNCHED();
    return TB_OK;
}

int attn_nsplit(int max_seq) { return (max_seq + kAttnTile - 1) / kAttnTile; }

int launch_attention(const DecState *st, const float *qkv, const float *kc, const float *vc,
                     float *part, float *out, uint32_t *xq, int hq, int hkv, int hd, int max_seq,
                     int cap, hipStream_t s) {
    TB_REQUIRE(cap >= 1, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: attention cap must be positive");
    const int ns = attn_nsplit(max_seq);
    TB_REQUIRE(ns <= kMaxTiles, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: max_seq_len above " + std::to_string(kMaxTiles * kAttnTile));
    const int G = hq / hkv;
    const float scale = 1.0f / sqrtf((float)hd);
    const size_t lds = sizeof(float) * ((size_t)G * hd + kAttnTile * (hd + 4) + kAttnTile * hd +
                                        G * kAttnTile + 2 * G);
    TB_REQUIRE(lds <= 160 * 1024, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: attention tile does not fit in LDS for this head layout");
    const int gp = G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : G <= 8 ? 8 : 0;
    if (gp && (hd == 128 || hd == 64)) {
        // at most kAttnMaxSplits blocks per KV head, each folding every
        // nb-th tile: the partials (and the merge) stay bounded for long caches
        const int nb = std::min(ns, kAttnMaxSplits);
#define TB_ATTN_REG(HD, GP)                                                                    \
    hipLaunchKernelGGL((k_attn_reg<HD, GP>), dim3(hkv, nb), dim3(256), 0, s, st, qkv, kc, vc, \
                       part, G, max_seq, nb, scale, cap)
        if (hd == 128) {
            if (gp == 1) TB_ATTN_REG(128, 1);
            else if (gp == 2) TB_ATTN_REG(128, 2);
            else if (gp == 4) TB_ATTN_REG(128, 4);
            else TB_ATTN_REG(128, 8);
            TB_LAUNCHED();
            hipLaunchKernelGGL(k_attn_merge_chunk<128>, dim3(hq, 4), dim3(64), 0, s, st, part, out,
                               xq, nb, cap);
        } else {
            if (gp == 1) TB_ATTN_REG(64, 1);
            else if (gp == 2) TB_ATTN_REG(64, 2);
            else if (gp == 4) TB_ATTN_REG(64, 4);
            else TB_ATTN_REG(64, 8);
            TB_LAUNCHED();
            hipLaunchKernelGGL(k_attn_merge_chunk<64>, dim3(hq, 2), dim3(64), 0, s, st, part, out,
                               xq, nb, cap);
        }
#undef TB_ATTN_REG
    } else if (hd == 128) {
        hipLaunchKernelGGL(k_attn<128>, dim3(hkv, ns), dim3(256), lds, s, st, qkv, kc, vc, part,
                           hq, hkv, max_seq, ns, scale, cap);
        TB_LAUNCHED();
        hipLaunchKernelGGL(k_attn_merge<128>, dim3(hq), dim3(64), 0, s, st, part, out, xq, ns,
                           cap);
    } else if (hd == 64) {
        hipLaunchKernelGGL(k_attn<64>, dim3(hkv, ns), dim3(256), lds, s, st, qkv, kc, vc, part,
                           hq, hkv, max_seq, ns, scale, cap);
        TB_LAUNCHED();
        hipLaunchKernelGGL(k_attn_merge<64>, dim3(hq), dim3(64), 0, s, st, part, out, xq, ns,
                           cap);
    } else {
        return fail(TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: head_dim must be 64 or 128");
    }
    TB_LAUNCHED();
    return TB_OK;
}

int launch_argmax(const float *logits, int n, float *pv, int *pi, DecState *st, int *history,
                  int hist_cap, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax_partial, dim3(kArgmaxBlocks), dim3(256), 0, s, logits, n, pv, pi);
    TB_LAUNCHED();
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s, pv, pi, kArgmaxBlocks, n, st,
                       history, hist_cap);
    TB_LAUNCHED();
    return TB_OK;
}

int launch_embed_rows(const int *tok, const float *embed, float *X, int M, int H, hipStream_t s) {
    hipLaunchKernelGGL(k_embed_rows, dim3(M), dim3(256), 0, s, tok, embed, X, H);
    TB_LAUNCHED();
    return TB_OK;
}

int launch_rmsnorm_rows(const float *X, const float *w, float *Xn, int M, int H, float eps,
                        hipStream_t s) {
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(M), dim3(256), 0, s, X, w, Xn, H, eps);
    TB_LAUNCHED();
    return TB_OK;
}

int launch_rope_rows(const float *qkv, float *q, float *kc, float *vc, const float *cos_t,
                     const float *sin_t, int start, int M, int hq, int hkv, int hd, int max_seq,
                     hipStream_t s) {
    const int nq = (hq + 2 * hkv) * hd;
    hipLaunchKernelGGL(k_rope_rows, dim3(M, hq + 2 * hkv), dim3(hd / 2), 0, s, qkv, nq, q, kc, vc,
                       cos_t, sin_t, start, hq, hkv, hd, max_seq);
    TB_LAUNCHED();
    return TB_OK;
}

namespace {

// Key groups per tile of the MFMA prefill attention: few rows share the four
// waves between row blocks and key groups.
int mfma_attn_kg(int M, int G) {
    const int nr = M * G;
    return nr <= 16 ? 4 : nr <= 32 ? 2 : 1;
}

// Key positions per tile for kg key groups: 32, or 64 for four key groups
// (each wave takes whole 16-key blocks).
int mfma_attn_tile(int kg) { return kg == 4 ? 64 : 32; }

template <int HD>
void launch_attn_mfma(int kg, dim3 grid, hipStream_t s, const float *q, const float *kc,
                      const float *vc, float *out, int start, int M, int hq, int hkv, int max_seq,
                      float scale, int tps, float *part, float *pml) {
#define TB_PA(KT, KG)                                                                         \
    hipLaunchKernelGGL((k_prefill_attn_mfma<HD, KT, KG>), grid, dim3(256), 0, s, q, kc, vc, out, \
                       start, M, hq, hkv, max_seq, scale, tps, part, pml)
    if (kg == 4) TB_PA(64, 4);
    else if (kg == 2) TB_PA(32, 2);
    else TB_PA(32, 1);
#undef TB_PA
}

}  // namespace

int prefill_attention_splits(int start, int M, int hq, int hkv) {
    // 64 / kg-row tiles; about 256 blocks (one or two per CU at their LDS;
    // TB_PREFILL_ATTN_BLOCKS overrides, measurement only), every split with at
    // least one key tile
    static const int target = [] {
        const char *e = getenv("TB_PREFILL_ATTN_BLOCKS");
        const int v = e ? atoi(e) : 0;
        return v > 0 ? v : 256;
    }();
    const int kg = mfma_attn_kg(M, hq / hkv);
    const int rows = 64 / kg, tile = mfma_attn_tile(kg);
    const int rtiles = (M * (hq / hkv) + rows - 1) / rows;
    const int tiles = (start + M - 1) / tile + 1;
    const int want = (target + rtiles * hkv - 1) / (rtiles * hkv);
    const int ns = std::max(1, std::min(want, tiles));
    const int tps = (tiles + ns - 1) / ns;
    return (tiles + tps - 1) / tps;
}

size_t prefill_attention_scratch(int M, int hq, int hd, int nsplit) {
    return nsplit > 1 ? (size_t)nsplit * M * hq * (hd + 2) * sizeof(float) : 0;
}

int launch_prefill_attention(const float *q, const float *kc, const float *vc, float *out,
                             int start, int M, int hq, int hkv, int hd, int max_seq,
                             float *scratch, hipStream_t s) {
    TB_REQUIRE(hkv > 0 && hq % hkv == 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: num_heads must be a multiple of num_kv_heads");
    TB_REQUIRE(hd == 64 || hd == 128, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: head_dim must be 64 or 128");
    const int kg = mfma_attn_kg(M, hq / hkv);
    const int kt = mfma_attn_tile(kg);
    const int nsplit = scratch ? prefill_attention_splits(start, M, hq, hkv) : 1;
    const int tiles = (start + M - 1) / kt + 1;
    const int tps = (tiles + nsplit - 1) / nsplit;
    float *part = nsplit > 1 ? scratch : nullptr;
    float *pml = nsplit > 1 ? scratch + (size_t)nsplit * M * hq * hd : nullptr;
    const int rows = 64 / kg;
    const int rtiles = (M * (hq / hkv) + rows - 1) / rows;
    const dim3 grid(rtiles, hkv, nsplit);
    const float scale = 1.0f / sqrtf((float)hd);
    if (hd == 128)
        launch_attn_mfma<128>(kg, grid, s, q, kc, vc, out, start, M, hq, hkv, max_seq, scale,
                              tps, part, pml);
    else
        launch_attn_mfma<64>(kg, grid, s, q, kc, vc, out, start, M, hq, hkv, max_seq, scale,
                             tps, part, pml);
    TB_LAUNCHED();
    if (nsplit > 1) {
        if (hd == 128)
            hipLaunchKernelGGL(k_prefill_merge<128>, dim3(M, hq), dim3(256), 0, s, part, pml, out,
                               M, hq, nsplit);
        else
            hipLaunchKernelGGL(k_prefill_merge<64>, dim3(M, hq), dim3(256), 0, s, part, pml, out,
                               M, hq, nsplit);
        TB_LAUNCHED();
    }
    return TB_OK;
}

}  // namespace tb

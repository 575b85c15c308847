// Token sampling on gfx950: repetition penalty, top-k, temperature softmax,
// nucleus (top-p) cut and one multinomial draw, without reading the logits
// back to the host.
//
// Replaces apply_repetition_penalty (src/llm/decoder.rs:878-899) and
// sample_logits (decoder.rs:908-1020):
//   * penalty: each distinct recent token's logit is divided by the penalty
//     when positive, multiplied otherwise (a bitmap over the vocabulary in LDS
//     makes "distinct" one atomicOr per token);
//   * greedy (temperature not finite or <= 0, or top_k <= 1) is the top-1;
//   * top-k: logits become order-preserving 32-bit keys (non-finite -> -inf);
//     each of NB blocks radix-selects the k-th largest key of its 2048-element
//     slice in LDS and writes its k best (ties: lower index first) in index
//     order; one block radix-selects the global top-k among those candidates;
//   * the k items are sorted (value descending, index ascending), p_i =
//     exp((v_i - v_0) / T), the nucleus keeps items while the mass before them
//     is <= top_p, and r = u * (kept mass) picks the first item whose running
//     mass reaches r.
// The reference draws u from an unseeded generator; here u comes from a
// counter-based generator (splitmix64 of seed + counter), so a seed fixes the
// stream.  The reference iterates its candidates unsorted; any fixed order
// gives the same distribution, and the sorted order makes the draw a function
// of u alone.
#include <math.h>

#include "decode.hpp"
#include "gemv_common.hpp"
#include "sample.hpp"
#include "tb_common.hpp"

namespace tb {

namespace {

constexpr int kThreads = 256;

// Order-preserving key of a logit.  Sampling treats every non-finite logit as
// -inf (decoder.rs:951-997); greedy keeps +inf (the reference's argmax compares
// raw values) and never picks a NaN past index 0.
__device__ __forceinline__ uint32_t fkey(float f, bool greedy) {
    if (greedy ? isnan(f) : !isfinite(f)) f = -INFINITY;
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float kval(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Exclusive prefix sum of a 0/1 flag over the block (256 threads, 4 waves),
// in thread order; *total gets the block's count.  Uses s[0..4].
__device__ __forceinline__ int block_excl(int flag, int *s, int *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const unsigned long long m = __ballot(flag);
    const int below = __popcll(m & ((1ull << lane) - 1ull));
    if (lane == 0) s[w] = __popcll(m);
    __syncthreads();
    int base = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        base += i < w ? s[i] : 0;
        tot += s[i];
    }
    __syncthreads();
    *total = tot;
    return base + below;
}

// The k-th largest (k >= 1, k <= n) of n keys, key_at(i) for i < n, over an
// NT-thread block; *need receives how many keys equal to it belong to the top
// k.  Eight passes of 4-bit digits from the top; each thread counts its keys
// per digit in registers (no atomics: logits crowd a few exponent digits, and
// LDS atomics on one bin serialise), the 16 counts are summed across the wave
// by a transpose reduction and across the waves through LDS (red: NT / 4
// floats; counts stay exact in f32 below 2^24).
template <int NT, class KeyAt>
__device__ uint32_t kth_largest(KeyAt key_at, int n, int k, float *red, int *need) {
    constexpr int NW = NT / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t prefix = 0u, mask = 0u;
    int kk = k;
    for (int shift = 28; shift >= 0; shift -= 4) {
        float c[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) c[j] = 0.f;
        for (int i = threadIdx.x; i < n; i += NT) {
            const uint32_t key = key_at(i);
            const bool act = (key & mask) == prefix;
            const uint32_t d = (key >> shift) & 15u;
#pragma unroll
            for (int j = 0; j < 16; ++j) c[j] += (act && d == (uint32_t)j) ? 1.f : 0.f;
        }
        gemv::transpose_reduce<16>(c, lane, 6);   // lane 4b: digit b's wave count
        if ((lane & 3) == 0) red[wave * 16 + ((lane >> 2) & 15)] = c[0];
        __syncthreads();
        int cum = 0, dsel = 0, rem = kk;
        for (int d = 15; d >= 0; --d) {
            int t = 0;
#pragma unroll
            for (int w = 0; w < NW; ++w) t += (int)red[w * 16 + d];
            if (cum + t >= kk) {
                dsel = d;
                rem = kk - cum;
                break;
            }
            cum += t;
        }
        prefix |= (uint32_t)dsel << shift;
        mask |= 15u << shift;
        kk = rem;
        __syncthreads();
    }
    *need = kk;
    return prefix;
}

// Writes, in index order, the keys > kth and the first `need` keys == kth
// (lowest positions) of keys[0..n) to ok/oi; returns the count (= k).
__device__ int gather_top(const uint32_t *keys, const int *idx, int n, uint32_t kth, int need,
                          uint32_t *ok, int *oi, int *s) {
    // (k <= kSampleMaxK items are taken; the bound below only guards ok / oi)
    int taken = 0, eq_seen = 0;
    for (int base = 0; base < n; base += kThreads) {
        const int i = base + threadIdx.x;
        const uint32_t key = i < n ? keys[i] : 0u;
        const int eq = (i < n && key == kth) ? 1 : 0;
        int eq_tot;
        const int eq_rank = eq_seen + block_excl(eq, s, &eq_tot);
        const int take = (i < n && (key > kth || (eq && eq_rank < need))) ? 1 : 0;
        int take_tot;
        const int pos = taken + block_excl(take, s, &take_tot);
        if (take && pos < kSampleMaxK) {
            ok[pos] = key;
            oi[pos] = idx ? idx[i] : i;
        }
        taken += take_tot;
        eq_seen += eq_tot;
    }
    return min(taken, kSampleMaxK);
}

__device__ __forceinline__ uint64_t splitmix(uint64_t x) {
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Penalty over the distinct tokens of `recent` (n of them, tokens outside the
// vocabulary skipped), in place.  One block; the vocabulary bitmap lives in LDS.
__global__ __launch_bounds__(kThreads) void k_penalty(float *__restrict__ logits, int V,
                                                      const int64_t *__restrict__ recent, int n,
                                                      const int *__restrict__ n_dev,
                                                      const SampleParams *__restrict__ prm) {
    extern __shared__ uint32_t bits[];
    const float pen = prm->penalty;
    if (n_dev) n = *n_dev;
    if (!(pen > 1.0f) || n <= 0) return;
    const int words = (V + 31) / 32;
    for (int i = threadIdx.x; i < words; i += kThreads) bits[i] = 0u;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kThreads) {
        const int64_t t = recent[i];
        if (t < 0 || t >= V) continue;
        const uint32_t bit = 1u << (t & 31);
        if ((atomicOr(&bits[t >> 5], bit) & bit) == 0u) {
            const float l = logits[t];
            logits[t] = l > 0.f ? l / pen : l * pen;
        }
    }
}

// Per-block top-k of a 2048-element slice: cand_key/idx [NB][kmax], cnt [NB].
__global__ __launch_bounds__(kThreads) void k_topk_slice(const float *__restrict__ logits, int V,
                                                         const SampleParams *__restrict__ prm,
                                                         uint32_t *__restrict__ cand_key,
                                                         int *__restrict__ cand_idx,
                                                         int *__restrict__ cnt) {
    __shared__ uint32_t keys[kSampleSlice];
    __shared__ uint32_t okey[kSampleMaxK];
    __shared__ int oidx[kSampleMaxK];
    __shared__ float red[kThreads / 4];
    __shared__ int sh[8];
    const int k = prm->k;
    if (k > kSampleMaxK) return;   // the large-k path samples
    const bool greedy = prm->greedy != 0;
    const int b = blockIdx.x, base = b * kSampleSlice;
    const int n = min(kSampleSlice, V - base);
    for (int i = threadIdx.x; i < n; i += kThreads) {
        const float v = logits[base + i];
        // greedy scans from logits[0] with strict > (decoder.rs:914-925): a NaN
        // there is never replaced, so it takes the largest key
        keys[i] = (greedy && base + i == 0 && isnan(v)) ? 0xFFFFFFFFu : fkey(v, greedy);
    }
    __syncthreads();
    const int kk = min(k, n);
    int need;
    const uint32_t kth =
        kth_largest<kThreads>([&](int i) { return keys[i]; }, n, kk, red, &need);
    const int m = gather_top(keys, nullptr, n, kth, need, okey, oidx, sh + 4);
    __syncthreads();
    for (int i = threadIdx.x; i < m; i += kThreads) {
        cand_key[(size_t)b * kSampleMaxK + i] = okey[i];
        cand_idx[(size_t)b * kSampleMaxK + i] = base + oidx[i];
    }
    if (threadIdx.x == 0) cnt[b] = m;
}

// Global top-k from the slices' candidates, the draw, and the result.
__global__ __launch_bounds__(kThreads) void k_topk_draw(const uint32_t *__restrict__ cand_key,
                                                        const int *__restrict__ cand_idx,
                                                        const int *__restrict__ cnt, int nb,
                                                        SampleParams *__restrict__ prm,
                                                        SampleOut *__restrict__ out,
                                                        DecState *__restrict__ st,
                                                        int *__restrict__ history, int hist_cap) {
    __shared__ uint32_t keys[kSampleCand];
    __shared__ int idx[kSampleCand];
    __shared__ uint32_t tk[kSampleMaxK];
    __shared__ int ti[kSampleMaxK];
    __shared__ float p[kSampleMaxK];
    __shared__ float red[kThreads / 4];
    __shared__ int sh[8];
    __shared__ int off[kSampleMaxBlocks + 1];
    const int k = prm->k;
    if (k > kSampleMaxK) return;   // the large-k path samples
    // slice offsets: an exclusive scan of the counts by wave 0 (nb <= 128)
    if (threadIdx.x < 64) {
        const int l = threadIdx.x;
        const int c0 = 2 * l < nb ? cnt[2 * l] : 0, c1 = 2 * l + 1 < nb ? cnt[2 * l + 1] : 0;
        int incl = c0 + c1;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(incl, o);
            if (l >= o) incl += t;
        }
        const int ex = incl - c0 - c1;
        if (2 * l < nb) off[2 * l] = ex;
        if (2 * l + 1 < nb) off[2 * l + 1] = ex + c0;
        if (l == 63) off[nb] = incl;
    }
    __syncthreads();
    const int n = off[nb];
    for (int e = threadIdx.x; e < nb * kSampleMaxK; e += kThreads) {
        const int b = e / kSampleMaxK, i = e - b * kSampleMaxK;
        if (i < cnt[b]) {
            keys[off[b] + i] = cand_key[e];
            idx[off[b] + i] = cand_idx[e];
        }
    }
    __syncthreads();
    const int kk = min(k, n);
    int need;
    const uint32_t kth =
        kth_largest<kThreads>([&](int i) { return keys[i]; }, n, kk, red, &need);
    const int m = gather_top(keys, idx, n, kth, need, tk, ti, sh + 4);
    // bitonic sort of the m (<= 128) items: key descending, index ascending
    for (int i = m + threadIdx.x; i < kSampleMaxK; i += kThreads) {
        tk[i] = 0u;
        ti[i] = 0x7FFFFFFF;
    }
    __syncthreads();
    for (int size = 2; size <= kSampleMaxK; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const int i = threadIdx.x;
            if (i < kSampleMaxK) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool desc = (i & size) == 0;
                    const uint32_t a = tk[i], c = tk[j];
                    const int ia = ti[i], ic = ti[j];
                    const bool a_first = a > c || (a == c && ia < ic);
                    if (a_first != desc) {
                        tk[i] = c; tk[j] = a;
                        ti[i] = ic; ti[j] = ia;
                    }
                }
            }
            __syncthreads();
        }
    if (threadIdx.x == 0) {
        int tok = ti[0];
        const float T = prm->temperature;
        float u = -1.f;
        if (!prm->greedy && m > 1) {
            const float vmax = kval(tk[0]), inv_t = 1.0f / T;
            float pre = 0.f;
            for (int i = 0; i < m; ++i) {
                p[i] = expf((kval(tk[i]) - vmax) * inv_t);
                pre += p[i];
            }
            int kept = m;
            const float tp = prm->top_p;
            if (tp > 0.f && tp < 1.f && pre > 0.f) {
                const float inv = 1.0f / pre;
                float cum = 0.f;
                for (int i = 0; i < m; ++i) {
                    if (cum > tp) {
                        kept = i;
                        break;
                    }
                    cum += p[i] * inv;
                }
            }
            float ks = 0.f;
            for (int i = 0; i < kept; ++i) ks += p[i];
            const uint64_t z = splitmix(prm->seed + (prm->counter + 1ull) * 0x9E3779B97F4A7C15ull);
            u = (float)(z >> 40) * 5.9604644775390625e-8f;   // [0, 1), 24 bits
            prm->counter += 1ull;
            const float r = u * ks;
            float acc = 0.f;
            for (int i = 0; i < kept; ++i) {
                acc += p[i];
                if (acc >= r) {
                    tok = ti[i];
                    break;
                }
            }
        }
        out->u = u;
        out->token = tok;
        out->kept = m;
        if (st) {   // the decoder's next step, as the greedy argmax tail does
            const int step = st->step;
            if (history && step < hist_cap) history[step] = tok;
            st->argmax = tok;
            st->token = tok;
            st->pos = st->pos + 1;
            st->step = step + 1;
        }
    }
}

// ---- top_k > kSampleMaxK: one block over the whole vocabulary ----
constexpr int kLargeThreads = 1024;

// Exclusive scan of one value per thread over an NT-thread block in thread
// order; *total gets the block's sum.  s: NT / 64 + 1 entries of LDS.
template <int NT, class T>
__device__ T block_scan_excl(T v, T *s, T *total) {
    constexpr int NW = NT / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    T incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const T t = __shfl_up(incl, o);
        if (lane >= o) incl += t;
    }
    if (lane == 63) s[wave] = incl;
    __syncthreads();
    if (threadIdx.x == 0) {
        T run = T(0);
        for (int w = 0; w < NW; ++w) {
            const T t = s[w];
            s[w] = run;
            run += t;
        }
        s[NW] = run;
    }
    __syncthreads();
    const T ex = s[wave] + incl - v;
    *total = s[NW];
    __syncthreads();
    return ex;
}

// The first item, in sorted order (key descending, then index ascending), at
// which the running mass of p crosses M (strict: > M, else >= M).  Items
// [0, n) are in index order.  Returns its position in the arrays (or -1 when
// the whole mass does not cross) and *through the mass up to and including it.
// The key of the crossing item comes from a radix search whose bins hold
// masses instead of counts, then its rank among equal keys from a block scan
// in index order.  red: NT / 4 floats; s: NT / 64 + 1 floats; si: 2 ints.
template <int NT>
__device__ int mass_cross(const uint32_t *keys, const float *p, int n, float M, bool strict,
                          float *red, float *s, int *si, float *through) {
    constexpr int NW = NT / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    auto crosses = [&](float x) { return strict ? x > M : x >= M; };
    uint32_t prefix = 0u, mask = 0u;
    float above = 0.f;   // mass of the items whose key is above the prefix
    for (int shift = 28; shift >= 0; shift -= 4) {
        float c[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) c[j] = 0.f;
        for (int i = threadIdx.x; i < n; i += NT) {
            const uint32_t key = keys[i];
            const bool act = (key & mask) == prefix;
            const uint32_t d = (key >> shift) & 15u;
            const float pi = p[i];
#pragma unroll
            for (int j = 0; j < 16; ++j) c[j] += (act && d == (uint32_t)j) ? pi : 0.f;
        }
        gemv::transpose_reduce<16>(c, lane, 6);
        if ((lane & 3) == 0) red[wave * 16 + ((lane >> 2) & 15)] = c[0];
        __syncthreads();
        int dsel = -1;
        for (int d = 15; d >= 0; --d) {
            float t = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) t += red[w * 16 + d];
            if (t > 0.f && crosses(above + t)) {
                dsel = d;
                break;
            }
            above += t;
        }
        __syncthreads();
        if (dsel < 0) {
            if (shift == 28) return -1;   // the whole mass stays on the near side of M
            // summation order left the cut in the last bin: take its lowest digit
            for (int d = 0; d < 16; ++d) {
                float t = 0.f;
                for (int w = 0; w < NW; ++w) t += red[w * 16 + d];
                if (t > 0.f) {
                    dsel = d;
                    break;
                }
            }
            dsel = dsel < 0 ? 0 : dsel;
        }
        prefix |= (uint32_t)dsel << shift;
        mask |= 15u << shift;
    }
    // the crossing item among those with key == prefix, in index order
    const int per = (n + NT - 1) / NT, lo = threadIdx.x * per, hi = min(n, lo + per);
    float part = 0.f;
    int last = -1;
    for (int i = lo; i < hi; ++i)
        if (keys[i] == prefix) {
            part += p[i];
            last = i;
        }
    float tot;
    const float base = block_scan_excl<NT, float>(part, s, &tot);
    if (threadIdx.x == 0) {
        si[0] = 0x7FFFFFFF;
        si[1] = -1;
    }
    __syncthreads();
    atomicMax(&si[1], last);   // the group's last item, when rounding never crosses
    float acc = above + base;
    for (int i = lo; i < hi; ++i)
        if (keys[i] == prefix) {
            acc += p[i];
            if (crosses(acc)) {
                atomicMin(&si[0], i);
                break;
            }
        }
    __syncthreads();
    const int pos = si[0] != 0x7FFFFFFF ? si[0] : si[1];
    // the mass through pos: recomputed by the thread whose range holds it
    if (pos >= lo && pos < hi) {
        float a = above + base;
        for (int i = lo; i <= pos; ++i)
            if (keys[i] == prefix) a += p[i];
        s[0] = a;
    }
    __syncthreads();
    *through = s[0];
    __syncthreads();
    return pos;
}

// Top-k sampling for k > kSampleMaxK: the k-th largest key over the whole
// vocabulary, the k items (in index order) into the scratch, p_i =
// exp((v_i - v_0) / T), the nucleus cut (the first item whose mass before it,
// normalised, exceeds top_p) and the draw (the first item whose running mass
// reaches u * the kept mass), both in sorted order, as the small-k path and
// the reference's sample_logits (decoder.rs:950-1019) visit them.  The masses
// are summed in a parallel order, so an item within an f32 rounding of the
// cut or the draw point may differ from a sequential sum's choice.
__global__ __launch_bounds__(kLargeThreads) void k_topk_large(
    const float *__restrict__ logits, int V, SampleParams *__restrict__ prm,
    uint32_t *__restrict__ ikey, int *__restrict__ iidx, float *__restrict__ ip,
    SampleOut *__restrict__ out, DecState *__restrict__ st, int *__restrict__ history,
    int hist_cap) {
    constexpr int NT = kLargeThreads, NW = NT / 64;
    __shared__ float red[NT / 4];
    __shared__ float sf[NW + 1];
    __shared__ int sn[NW + 1];
    __shared__ int si[2];
    __shared__ uint32_t smax[2];
    const int k = prm->k;
    if (k <= kSampleMaxK) return;   // the small-k kernels sample
    const int kk = min(k, V);
    int need;
    const uint32_t kth = kth_largest<NT>([&](int i) { return fkey(logits[i], false); }, V, kk,
                                         red, &need);
    // the k items in index order: each thread a contiguous range of the vocabulary
    const int per = (V + NT - 1) / NT, lo = threadIdx.x * per, hi = min(V, lo + per);
    int ng = 0, ne = 0;
    for (int i = lo; i < hi; ++i) {
        const uint32_t key = fkey(logits[i], false);
        ng += key > kth;
        ne += key == kth;
    }
    int tot;
    const int eq_base = block_scan_excl<NT, int>(ne, sn, &tot);
    const int eq_take = max(0, min(ne, need - eq_base));
    const int base = block_scan_excl<NT, int>(ng + eq_take, sn, &tot);
    int w = base, eq_seen = 0;
    for (int i = lo; i < hi; ++i) {
        const uint32_t key = fkey(logits[i], false);
        const bool eq = key == kth;
        if (key > kth || (eq && eq_seen < eq_take)) {
            ikey[w] = key;
            iidx[w] = i;
            ++w;
        }
        eq_seen += eq;
    }
    __syncthreads();
    const int n = tot;   // == kk
    // the top item: the largest key, lowest index among equals (items in index order)
    if (threadIdx.x == 0) smax[0] = 0u;
    __syncthreads();
    uint32_t mk = 0u;
    for (int i = threadIdx.x; i < n; i += NT) mk = max(mk, ikey[i]);
    atomicMax(&smax[0], mk);
    __syncthreads();
    const uint32_t kmax = smax[0];
    if (threadIdx.x == 0) si[0] = 0x7FFFFFFF;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += NT)
        if (ikey[i] == kmax) atomicMin(&si[0], i);
    __syncthreads();
    const int top = si[0];
    __syncthreads();
    const float T = prm->temperature, inv_t = 1.0f / T, vmax = kval(kmax);
    float part = 0.f;
    for (int i = threadIdx.x; i < n; i += NT) {
        const float pi = expf((kval(ikey[i]) - vmax) * inv_t);
        ip[i] = pi;
        part += pi;
    }
    __syncthreads();
    float pre;
    (void)block_scan_excl<NT, float>(part, sf, &pre);
    float ks = pre;
    const float tp = prm->top_p;
    if (tp > 0.f && tp < 1.f && n > 1 && pre > 0.f) {
        float thr;
        const int c = mass_cross<NT>(ikey, ip, n, tp * pre, true, red, sf, si, &thr);
        if (c >= 0) ks = thr;
    }
    const uint64_t z = splitmix(prm->seed + (prm->counter + 1ull) * 0x9E3779B97F4A7C15ull);
    const float u = (float)(z >> 40) * 5.9604644775390625e-8f;   // [0, 1), 24 bits
    float dthr;
    const int d = mass_cross<NT>(ikey, ip, n, u * ks, false, red, sf, si, &dthr);
    if (threadIdx.x == 0) {
        const int tok = iidx[d >= 0 ? d : top];
        prm->counter += 1ull;
        out->u = u;
        out->token = tok;
        out->kept = n;
        if (st) {   // the decoder's next step, as the greedy argmax tail does
            const int step = st->step;
            if (history && step < hist_cap) history[step] = tok;
            st->argmax = tok;
            st->token = tok;
            st->pos = st->pos + 1;
            st->step = step + 1;
        }
    }
}

// Pushes the step's input token onto the recent-token window (the last
// kSampleWindow tokens, decoder.rs:859-876) before its penalty is applied.
__global__ void k_window_push(const DecState *__restrict__ st, SampleWindow *__restrict__ w) {
    if (threadIdx.x != 0) return;
    int n = w->n;
    if (n == kSampleWindow) {
        for (int i = 1; i < kSampleWindow; ++i) w->tok[i - 1] = w->tok[i];
        n -= 1;
    }
    w->tok[n] = st->token;
    w->n = n + 1;
}

}  // namespace

float sample_uniform(uint64_t seed, uint64_t counter) {
    uint64_t x = seed + (counter + 1ull) * 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    x ^= x >> 31;
    return (float)(x >> 40) * 5.9604644775390625e-8f;
}

int sample_blocks(int V) { return (V + kSampleSlice - 1) / kSampleSlice; }

int launch_sample(float *logits, int V, const int64_t *recent, int n_recent,
                  SampleParams *prm, const SampleScratch &ws, SampleOut *out, hipStream_t st,
                  bool large, SampleWindow *win, DecState *dstate, int *history, int hist_cap) {
    const int nb = sample_blocks(V);
    TB_REQUIRE(nb <= kSampleMaxBlocks, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: device sampling supports vocabularies up to " +
                   std::to_string(kSampleMaxBlocks * kSampleSlice));
    const size_t lds = (size_t)((V + 31) / 32) * 4;
    TB_REQUIRE(lds <= 64 * 1024, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: repetition penalty bitmap exceeds LDS");
    if (win) {
        hipLaunchKernelGGL(k_window_push, dim3(1), dim3(64), 0, st, dstate, win);
        TB_LAUNCHED();
        hipLaunchKernelGGL(k_penalty, dim3(1), dim3(kThreads), lds, st, logits, V, win->tok, 0,
                           &win->n, prm);
        TB_LAUNCHED();
    } else if (recent && n_recent > 0) {
        hipLaunchKernelGGL(k_penalty, dim3(1), dim3(kThreads), lds, st, logits, V, recent,
                           n_recent, (const int *)nullptr, prm);
        TB_LAUNCHED();
    }
    if (large) {
        hipLaunchKernelGGL(k_topk_large, dim3(1), dim3(kLargeThreads), 0, st, logits, V, prm,
                           ws.key, ws.idx, ws.p, out, dstate, history, hist_cap);
        TB_LAUNCHED();
        return TB_OK;
    }
    hipLaunchKernelGGL(k_topk_slice, dim3(nb), dim3(kThreads), 0, st, logits, V, prm, ws.key,
                       ws.idx, ws.cnt);
    TB_LAUNCHED();
    hipLaunchKernelGGL(k_topk_draw, dim3(1), dim3(kThreads), 0, st, ws.key, ws.idx, ws.cnt, nb,
                       prm, out, dstate, history, hist_cap);
    TB_LAUNCHED();
    return TB_OK;
}

}  // namespace tb

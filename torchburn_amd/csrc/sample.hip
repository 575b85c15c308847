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

// The k-th largest (k >= 1) of the n keys in LDS; *need receives how many keys
// equal to it belong to the top k.  hist: 256 ints of LDS; sh: 2 ints.
__device__ uint32_t kth_largest(const uint32_t *keys, int n, int k, int *hist, int *sh,
                                int *need) {
    uint32_t prefix = 0u, mask = 0u;
    int kk = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = threadIdx.x; i < 256; i += kThreads) hist[i] = 0;
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += kThreads) {
            const uint32_t key = keys[i];
            if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            int cum = 0, d = 255;
            for (; d > 0; --d) {
                if (cum + hist[d] >= kk) break;
                cum += hist[d];
            }
            sh[0] = d;
            sh[1] = kk - cum;
        }
        __syncthreads();
        prefix |= (uint32_t)sh[0] << shift;
        mask |= 255u << shift;
        kk = sh[1];
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
    __shared__ int hist[256];
    __shared__ int sh[8];
    const int k = prm->k;
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
    const uint32_t kth = kth_largest(keys, n, kk, hist, sh, &need);
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
    __shared__ int hist[256];
    __shared__ int sh[8];
    __shared__ int off[kSampleMaxBlocks + 1];
    const int k = prm->k;
    if (threadIdx.x == 0) {
        int o = 0;
        for (int b = 0; b < nb; ++b) {
            off[b] = o;
            o += cnt[b];
        }
        off[nb] = o;
    }
    __syncthreads();
    const int n = off[nb];
    for (int b = 0; b < nb; ++b)
        for (int i = threadIdx.x; i < cnt[b]; i += kThreads) {
            keys[off[b] + i] = cand_key[(size_t)b * kSampleMaxK + i];
            idx[off[b] + i] = cand_idx[(size_t)b * kSampleMaxK + i];
        }
    __syncthreads();
    const int kk = min(k, n);
    int need;
    const uint32_t kth = kth_largest(keys, n, kk, hist, sh, &need);
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
                  SampleWindow *win, DecState *dstate, int *history, int hist_cap) {
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
    hipLaunchKernelGGL(k_topk_slice, dim3(nb), dim3(kThreads), 0, st, logits, V, prm, ws.key,
                       ws.idx, ws.cnt);
    TB_LAUNCHED();
    hipLaunchKernelGGL(k_topk_draw, dim3(1), dim3(kThreads), 0, st, ws.key, ws.idx, ws.cnt, nb,
                       prm, out, dstate, history, hist_cap);
    TB_LAUNCHED();
    return TB_OK;
}

}  // namespace tb

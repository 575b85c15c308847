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
//   * top-k: logits become order-preserving 32-bit keys (non-finite -> -inf),
//     packed with their index into 64-bit items that order as the sampler
//     does (key descending, then index ascending); for k <= kSampleMaxK every
//     wave of a wide launch lists its best 8 items, one block takes the items
//     at or above the k-th best wave maximum and ranks them (k_topk_select);
//     for larger k one block radix-selects over the whole vocabulary;
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
    const bool drop = greedy ? isnan(f) : !isfinite(f);
    const uint32_t b = drop ? 0xFF800000u : __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float kval(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// The key the sampler ranks logit v at index id by.  Greedy scans from
// logits[0] with strict > (decoder.rs:914-925): a NaN there is never
// replaced, so it takes the largest key.
__device__ __forceinline__ uint32_t sample_key(float v, int id, bool greedy) {
    return (greedy && id == 0 && isnan(v)) ? 0xFFFFFFFFu : fkey(v, greedy);
}

// An item: key in the high word, the complement of the index in the low word,
// so that larger items come first in the sampler's order.  0 is no item.
__device__ __forceinline__ uint64_t pack_item(uint32_t key, int id) {
    return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)id);
}
__device__ __forceinline__ uint32_t item_key(uint64_t it) { return (uint32_t)(it >> 32); }
__device__ __forceinline__ int item_index(uint64_t it) {
    return (int)(0xFFFFFFFFu - (uint32_t)it);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    const int lo = __shfl_xor((int)(uint32_t)v, m);
    const int hi = __shfl_xor((int)(uint32_t)(v >> 32), m);
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
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

__device__ __forceinline__ uint64_t splitmix(uint64_t x) {
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Penalty over the distinct tokens of `recent` (n of them, tokens outside the
// vocabulary skipped), in place.  With `win`, the step's input token is first
// pushed onto the recent-token window (the last kSampleWindow tokens,
// decoder.rs:859-876) and the penalty covers the window.  One block; a
// vocabulary bitmap in LDS (only the words the tokens touch are cleared) makes
// "distinct" one atomicOr per token.
__global__ __launch_bounds__(kThreads) void k_penalty(float *__restrict__ logits, int V,
                                                      const int64_t *recent, int n,
                                                      SampleWindow *__restrict__ win,
                                                      const DecState *__restrict__ dstate,
                                                      const SampleParams *__restrict__ prm) {
    extern __shared__ uint32_t bits[];
    __shared__ int64_t wtok[kSampleWindow];
    const int tid = threadIdx.x;
    if (win) {   // push onto the ring, then the live slots are the window
        const int c = win->n, head = win->head;
        const int slot = c < kSampleWindow ? (head + c) % kSampleWindow : head;
        if (tid < kSampleWindow)
            wtok[tid] = tid == slot ? (int64_t)dstate->token : win->tok[tid];
        __syncthreads();   // every thread read the ring before thread 0 changes it
        if (tid == 0) {
            win->tok[slot] = wtok[slot];
            win->head = c < kSampleWindow ? head : (head + 1) % kSampleWindow;
            win->n = c < kSampleWindow ? c + 1 : c;
        }
        // the live slots: all of them once full, else slots head .. head + c
        n = c < kSampleWindow ? c + 1 : kSampleWindow;
        if (n < kSampleWindow && tid < kSampleWindow) {
            const int rel = (tid - head + kSampleWindow) % kSampleWindow;
            if (rel >= n) wtok[tid] = -1;   // not live: skipped below
        }
        __syncthreads();
        recent = wtok;
        n = kSampleWindow;
    }
    const float pen = prm->penalty;
    if (!(pen > 1.0f) || n <= 0) return;
    for (int i = tid; i < n; i += kThreads) {
        const int64_t t = recent[i];
        if (t >= 0 && t < V) bits[t >> 5] = 0u;
    }
    __syncthreads();
    for (int i = tid; i < n; i += kThreads) {
        const int64_t t = recent[i];
        if (t < 0 || t >= V) continue;
        const uint32_t bit = 1u << (t & 31);
        if ((atomicOr(&bits[t >> 5], bit) & bit) == 0u) {
            const float l = logits[t];
            logits[t] = l > 0.f ? l / pen : l * pen;
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

// The top items of n keys given the k-th largest key kth and how many keys
// equal to it belong (need): emit(w, key, i) for the keys above kth and the
// first `need` equal to it, w = 0, 1, ... in index order (each thread takes a
// contiguous range of the indices).  Returns the count.  sn: NT / 64 + 1 ints.
template <int NT, class KeyAt, class Emit>
__device__ int gather_top(KeyAt key_at, int n, uint32_t kth, int need, int *sn, Emit emit) {
    const int per = (n + NT - 1) / NT, lo = min(n, (int)threadIdx.x * per), hi = min(n, lo + per);
    int ng = 0, ne = 0;
    for (int i = lo; i < hi; ++i) {
        const uint32_t key = key_at(i);
        ng += key > kth;
        ne += key == kth;
    }
    int tot;
    const int eq_base = block_scan_excl<NT, int>(ne, sn, &tot);
    const int eq_take = max(0, min(ne, need - eq_base));
    const int base = block_scan_excl<NT, int>(ng + eq_take, sn, &tot);
    int w = base, eq_seen = 0;
    for (int i = lo; i < hi; ++i) {
        const uint32_t key = key_at(i);
        const bool eq = key == kth;
        if (key > kth || (eq && eq_seen < eq_take)) emit(w++, key, i);
        eq_seen += eq;
    }
    __syncthreads();
    return tot;
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
    const int n = gather_top<NT>([&](int i) { return fkey(logits[i], false); }, V, kth, need, sn,
                                 [&](int w, uint32_t key, int i) {
                                     ikey[w] = key;
                                     iidx[w] = i;
                                 });   // == kk
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

// ---- top_k <= kSampleMaxK: wave lists, a threshold, ranks ----
//
// k_topk_lists (nb = ceil(V / 2048) blocks of 4 waves, 8 ids per lane): the
// vocabulary is cut into runs of kRun ids; block b takes runs b, b + nb,
// b + 2 nb, ..., and in each run wave w takes the ids = w (mod 4), so a
// wave's 512 ids are spread over the vocabulary and neighbouring ids (which
// related tokens often are) fall to different waves.  Each wave writes its
// best q = min(k, kListQ) items, best first (0 past its count), and its count.
//
// k_topk_select (one block): the pool is the best j = ceil(k / W) listed
// items of each of the W waves; T = the k-th best of the pool (every item
// when the pool holds fewer than k).  At least k items are >= T, so the top k
// all are.  The candidates are the listed items >= T; a candidate's rank
// among them is its place in the sorted order.  A wave whose q-th item ranks
// before the (m-1)-th candidate may hold more of the top m than it listed; if
// one does, its ids are read again and those of its items at or above the
// m-th candidate that it did not list join.  The candidates' top m is then the
// global top m: a top item x missing from the lists sits below its wave's q
// listed items, all of which lie above x, so above the m-th best item, so
// above the m-th candidate, and the rescan takes x.  Past kCandCap
// candidates, an exact radix select over the vocabulary takes over.
constexpr int kRun = 16;
constexpr int kListQ = 8;
constexpr int kCandCap = 2048;
constexpr int kPoolCap = kSampleLists + kSampleMaxK + 8;   // W * ceil(k / W) < W + k, + 8 zeros
constexpr int kSelThreads = 1024;
constexpr int kMaxFlagged = kSampleMaxK / kListQ;
static_assert(kSampleLists * kListQ * 8 <= kSampleCand * 4, "wave lists fit the key scratch");

// Blocks of the list kernel (2048 ids each: 4 waves x 64 lanes x kListQ).
inline int list_blocks(int V) { return (V + 2047) / 2048; }

// The id that item i of lane l in wave w of block b (of nb) stands for; ids
// >= V are no item.
__device__ __forceinline__ int list_id(int b, int nb, int w, int l, int i) {
    return kRun * (b + nb * ((l >> 2) + 16 * i)) + 4 * (l & 3) + w;
}

__device__ __forceinline__ void cas_desc(uint64_t &a, uint64_t &b) {
    const uint64_t x = a, y = b;
    const bool s = x < y;
    a = s ? y : x;
    b = s ? x : y;
}

// Batcher's odd-even merge network over 8 items, best first.
__device__ __forceinline__ void sort8_desc(uint64_t (&v)[8]) {
    cas_desc(v[0], v[1]); cas_desc(v[2], v[3]); cas_desc(v[4], v[5]); cas_desc(v[6], v[7]);
    cas_desc(v[0], v[2]); cas_desc(v[1], v[3]); cas_desc(v[4], v[6]); cas_desc(v[5], v[7]);
    cas_desc(v[1], v[2]); cas_desc(v[5], v[6]);
    cas_desc(v[0], v[4]); cas_desc(v[1], v[5]); cas_desc(v[2], v[6]); cas_desc(v[3], v[7]);
    cas_desc(v[2], v[4]); cas_desc(v[3], v[5]);
    cas_desc(v[1], v[2]); cas_desc(v[3], v[4]); cas_desc(v[5], v[6]);
}

// x from another lane of the same row or the row before, by a DPP move
// (lanes outside row_mask keep old).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t old, uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)x, CTRL, ROW_MASK, 0xF, false);
}

// The wave's maximum, uniform: quad swaps and row mirrors leave every lane
// with its 16-lane row's maximum, row broadcasts carry rows 0-2 into row 3,
// and lane 63 is read.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
    x = max(x, dpp_u32<0xB1, 0xF>(x, x));    // quad_perm [1,0,3,2]
    x = max(x, dpp_u32<0x4E, 0xF>(x, x));    // quad_perm [2,3,0,1]
    x = max(x, dpp_u32<0x141, 0xF>(x, x));   // row_half_mirror
    x = max(x, dpp_u32<0x140, 0xF>(x, x));   // row_mirror
    x = max(x, dpp_u32<0x142, 0xA>(x, x));   // row_bcast:15 into rows 1 and 3
    x = max(x, dpp_u32<0x143, 0xC>(x, x));   // row_bcast:31 into rows 2 and 3
    return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}

// The wave's best item among the lanes' x (0: none), uniform: the best key,
// then, only when several lanes hold it, the best index among them.
__device__ __forceinline__ uint64_t wave_best(uint64_t x) {
    const uint32_t hk = (uint32_t)(x >> 32), mk = wave_max_u32(hk);
    const unsigned long long at = __ballot(hk == mk && x != 0ull);
    if (__popcll(at) == 1) {
        const int src = __ffsll((long long)at) - 1;
        return ((uint64_t)mk << 32) | (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, src);
    }
    const uint32_t ml = wave_max_u32(hk == mk ? (uint32_t)x : 0u);
    return ((uint64_t)mk << 32) | ml;
}

// With `win` (the decoder's step), the repetition penalty of the window as it
// stands after the step's input token (dstate->token) is pushed: every block
// finds the distinct window tokens it holds (the inverse of list_id), and the
// thread holding one divides or multiplies its copy (decoder.rs:878-899) and
// writes it back, so the select kernel's re-reads see it.  The push itself is
// the select kernel's, after every block here has read the ring.
__global__ __launch_bounds__(kThreads) void k_topk_lists(float *__restrict__ logits, int V,
                                                         const SampleParams *__restrict__ prm,
                                                         uint64_t *__restrict__ lists,
                                                         int *__restrict__ wcnt,
                                                         const SampleWindow *__restrict__ win,
                                                         const DecState *__restrict__ dstate) {
    __shared__ int pen_n;
    __shared__ int pen_e[kSampleWindow + 1];
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63, nb = gridDim.x;
    float x[kListQ];
    int n = 0;
#pragma unroll
    for (int i = 0; i < kListQ; ++i) {   // every load issued at once (ids past V read logits[V-1])
        const int id = list_id(blockIdx.x, nb, w, l, i);
        x[i] = logits[min(id, V - 1)];
        n += __popcll(__ballot(id < V));
    }
    if (win) {
        const float pen = prm->penalty;
        if (threadIdx.x == 0) pen_n = 0;
        __syncthreads();
        if (w == 0 && pen > 1.0f) {
            // lane l: ring slot l if live after the push; the pushed token
            // replaces the slot it lands in (the oldest one when full)
            const int c = win->n, head = win->head;
            const int slot = c < kSampleWindow ? (head + c) % kSampleWindow : head;
            const int live_n = c < kSampleWindow ? c + 1 : kSampleWindow;
            const int64_t tin = dstate->token;
            const int64_t t = l == slot ? tin : win->tok[l];
            const bool live = (l - head + kSampleWindow) % kSampleWindow < live_n;
            const bool ok = live && t >= 0 && t < V;
            const int r = ok ? (int)(t / kRun) : 0, o = ok ? (int)(t % kRun) : 0;
            const bool own = ok && r % nb == (int)blockIdx.x;
            unsigned long long ob = __ballot(own);
            while (ob) {   // usually none or one: 64 tokens over nb blocks
                const int j = __ffsll((long long)ob) - 1;
                ob &= ob - 1ull;
                const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)t, j);
                const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)t >> 32), j);
                const int64_t tj = (int64_t)(((uint64_t)hi << 32) | lo);
                // the first live slot holding tj applies it
                if (__ballot(ok && l < j && t == tj) == 0ull && l == j) {
                    const int jj = r / nb;
                    const int e = ((o & 3) << 16) | ((((jj & 15) << 2) | (o >> 2)) << 8) | (jj >> 4);
                    pen_e[atomicAdd(&pen_n, 1)] = e;
                }
            }
        }
        __syncthreads();
        const int ne = pen_n;
        for (int ei = 0; ei < ne; ++ei) {
            const int e = pen_e[ei];
            if ((e >> 16) != w || ((e >> 8) & 255) != l) continue;
            const int item = e & 255;
#pragma unroll
            for (int i = 0; i < kListQ; ++i)
                if (i == item) {
                    const float v = x[i];
                    x[i] = v > 0.f ? v / pen : v * pen;
                    logits[list_id(blockIdx.x, nb, w, l, i)] = x[i];
                }
        }
    }
    // (the k test comes last, so that the loads above need not wait for it)
    const int k = prm->k;
    const bool greedy = prm->greedy != 0;
    const int q = min(k, kListQ);
    uint64_t v[kListQ];
#pragma unroll
    for (int i = 0; i < kListQ; ++i) {
        const int id = list_id(blockIdx.x, nb, w, l, i);
        const uint64_t it = pack_item(sample_key(x[i], id, greedy), id);
        v[i] = id < V ? it : 0ull;
    }
    sort8_desc(v);
    // q rounds: the wave's best head leaves its lane (items are distinct)
    uint64_t mine = 0ull;
    for (int t = 0; t < q; ++t) {
        const uint64_t best = wave_best(v[0]);
        if (l == t) mine = best;
        if (best != 0ull && v[0] == best) {
#pragma unroll
            for (int i = 0; i + 1 < kListQ; ++i) v[i] = v[i + 1];
            v[kListQ - 1] = 0ull;
        }
    }
    if (k > kSampleMaxK) return;   // the large-k path samples
    const int gw = blockIdx.x * 4 + w;
    if (l < kListQ) lists[(size_t)gw * kListQ + l] = mine;
    if (l == 0) wcnt[gw] = n;
}

// Appends `it` (and tag) where keep holds to buf / tags (positions from
// *count; past cap only counted).  Called by every active lane of a wave.
__device__ __forceinline__ void wave_append(bool keep, uint64_t it, int tag, uint64_t *buf,
                                            int *tags, int cap, int *count) {
    const unsigned long long b = __ballot(keep);
    if (b == 0ull) return;
    const int lane = threadIdx.x & 63, leader = __ffsll((long long)b) - 1;
    int base = 0;
    if (lane == leader) base = atomicAdd(count, __popcll(b));
    base = __shfl(base, leader);
    if (keep) {
        const int pos = base + __popcll(b & ((1ull << lane) - 1ull));
        if (pos < cap) {
            buf[pos] = it;
            if (tags) tags[pos] = tag;
        }
    }
}

// rank[c] += how many of a[0..n) are greater than a[c] (rank zero on entry):
// a holds distinct nonzero items and zeros up to the next multiple of 8
// (16-byte aligned).  Each wave takes 64 items against a share of a (waves
// left over split a between them and add their counts); ends with a barrier.
template <int NT>
__device__ void rank_items(const uint64_t *a, int n, int *rank) {
    constexpr int NW = NT / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int groups = (n + 63) / 64, parts = groups >= NW ? 1 : NW / groups;
    const int n8 = (n + 7) & ~7, chunk = ((n8 + parts - 1) / parts + 7) & ~7;
    for (int u = wave; u < groups * parts; u += NW) {
        const int g = u / parts, pt = u - g * parts, c = g * 64 + lane;
        const uint64_t me = c < n ? a[c] : ~0ull;
        const int j1 = min(n8, (pt + 1) * chunk);
        int r = 0;
        for (int j = pt * chunk; j < j1; j += 8) {
            const ulonglong2 x0 = *reinterpret_cast<const ulonglong2 *>(a + j);
            const ulonglong2 x1 = *reinterpret_cast<const ulonglong2 *>(a + j + 2);
            const ulonglong2 x2 = *reinterpret_cast<const ulonglong2 *>(a + j + 4);
            const ulonglong2 x3 = *reinterpret_cast<const ulonglong2 *>(a + j + 6);
            r += (x0.x > me) + (x0.y > me) + (x1.x > me) + (x1.y > me) + (x2.x > me) +
                 (x2.y > me) + (x3.x > me) + (x3.y > me);
        }
        if (c < n && r) atomicAdd(&rank[c], r);
    }
    __syncthreads();
}

__global__ __launch_bounds__(kSelThreads) void k_topk_select(
    const float *__restrict__ logits, int V, int nb, const uint64_t *__restrict__ lists,
    const int *__restrict__ wcnt, SampleParams *__restrict__ prm, SampleOut *__restrict__ out,
    DecState *__restrict__ st, int *__restrict__ history, int hist_cap,
    SampleWindow *__restrict__ win) {
    constexpr int NT = kSelThreads, NW = NT / 64;
    constexpr int kPer = kSampleLists * kListQ / NT;   // list slots per thread
    __shared__ __align__(16) uint64_t cand[kCandCap];
    __shared__ int ctag[kCandCap];
    __shared__ int crank[kCandCap];
    __shared__ uint64_t top[kSampleMaxK];
    // the pool and its ranks, then (once T is known) the draw's masses
    constexpr int kPoolBytes = kPoolCap * 12, kDrawBytes = 3 * kSampleMaxK * 4;
    __shared__ __align__(16) unsigned char scratch[kPoolBytes > kDrawBytes ? kPoolBytes : kDrawBytes];
    uint64_t *pool = reinterpret_cast<uint64_t *>(scratch);
    int *prank = reinterpret_cast<int *>(scratch + kPoolCap * 8);
    float *p = reinterpret_cast<float *>(scratch);
    float *cp = p + kSampleMaxK;
    float *cb = cp + kSampleMaxK;
    __shared__ float red[NT / 4];
    __shared__ int sn[NW + 1];
    __shared__ int flagged[kMaxFlagged];
    __shared__ uint64_t s_t;
    __shared__ int n_cand, n_pool, n_flag, s_lim;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int W = 4 * nb, slots = W * kListQ;
    uint64_t li[kPer];
    int lc[kPer];
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        const int e = tid + r * NT;
        li[r] = e < slots ? lists[e] : 0ull;
        lc[r] = e < slots ? wcnt[e / kListQ] : 0;
    }
    const int k = prm->k;
    if (k > kSampleMaxK) return;   // the large-k path samples
    const bool greedy = prm->greedy != 0;
    const int q = min(k, kListQ), m = min(k, V), jp = min(q, (k + W - 1) / W);
    if (tid == 0) {
        n_cand = 0;
        n_pool = 0;
        n_flag = 0;
        s_t = 1ull;   // every item
    }
    for (int i = tid; i < kCandCap; i += NT) crank[i] = 0;
    for (int i = tid; i < kPoolCap; i += NT) prank[i] = 0;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        const int e = tid + r * NT;
        wave_append(li[r] != 0ull && (e & (kListQ - 1)) < jp, li[r], 0, pool, nullptr,
                    kPoolCap - 8, &n_pool);
    }
    __syncthreads();
    const int np = n_pool;
    if (np >= k) {   // T = the k-th best of the pool
        if (tid < 8) pool[np + tid] = 0ull;   // np + 8 <= kPoolCap
        __syncthreads();
        rank_items<NT>(pool, np, prank);
        for (int c = tid; c < np; c += NT)
            if (prank[c] == k - 1) s_t = pool[c];
        __syncthreads();
    }
    const uint64_t T = s_t;
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        const int e = tid + r * NT, slot = e & (kListQ - 1);
        const int tag = (slot == q - 1 && lc[r] > q) ? e / kListQ : -1;
        wave_append(li[r] >= T && slot < q, li[r], tag, cand, ctag, kCandCap, &n_cand);
    }
    __syncthreads();
    int nc = n_cand;
    // ranks -> top[0..m); a short wave's q-th item ranked before m - 1 flags it
    auto order = [&](bool flags) {
        if (tid < 8) cand[nc + tid] = 0ull;   // nc + 8 <= kCandCap: see callers
        if (!flags)
            for (int c = tid; c < nc; c += NT) crank[c] = 0;
        __syncthreads();
        rank_items<NT>(cand, nc, crank);
        for (int c = tid; c < nc; c += NT) {
            const int r = crank[c];
            if (r < m) top[r] = cand[c];
            if (flags && ctag[c] >= 0 && r < m - 1) {
                const int f = atomicAdd(&n_flag, 1);
                if (f < kMaxFlagged) flagged[f] = ctag[c];
            }
        }
        __syncthreads();
    };
    bool exact = nc > kCandCap - 8;
    if (!exact) {
        order(true);
        const int nf = n_flag;
        if (nf > kMaxFlagged) {
            exact = true;
        } else if (nf > 0) {
            const uint64_t thr = nc >= m ? top[m - 1] : 1ull;
            for (int f = wave; f < nf; f += NW) {
                const int L = flagged[f], b = L >> 2, w = L & 3;
                const uint64_t last = lists[(size_t)L * kListQ + q - 1];
                for (int i = 0; i < kListQ; ++i) {
                    const int id = list_id(b, nb, w, lane, i);
                    const uint64_t it =
                        id < V ? pack_item(sample_key(logits[id], id, greedy), id) : 0ull;
                    wave_append(it < last && it >= thr, it, -1, cand, ctag, kCandCap, &n_cand);
                }
            }
            __syncthreads();
            nc = n_cand;
            exact = nc > kCandCap - 8;
            if (!exact) order(false);
        }
    }
    if (exact) {   // the m best over the whole vocabulary, then their order
        int need;
        const uint32_t kth = kth_largest<NT>(
            [&](int i) { return sample_key(logits[i], i, greedy); }, V, m, red, &need);
        nc = gather_top<NT>([&](int i) { return sample_key(logits[i], i, greedy); }, V, kth, need,
                            sn, [&](int w, uint32_t key, int i) { cand[w] = pack_item(key, i); });
        order(false);
    }
    // the draw over top[0..m), in order; sums run in sequence, as the
    // reference's loops do, and the nucleus step is not contracted
    const bool draw = !greedy && m > 1;
    if (draw) {
        const float vmax = kval(item_key(top[0])), inv_t = 1.0f / prm->temperature;
        for (int i = tid; i < kSampleMaxK; i += NT)
            p[i] = i < m ? expf((kval(item_key(top[i])) - vmax) * inv_t) : 0.f;
        __syncthreads();
        if (tid == 0) {   // running masses in chunks of 16, the next chunk's loads in flight
            const float4 *p4 = reinterpret_cast<const float4 *>(p);
            float4 *cp4 = reinterpret_cast<float4 *>(cp);
            float4 *cb4 = reinterpret_cast<float4 *>(cb);
            float4 a[4], nx[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) a[t] = p4[t];
            float pre = 0.f;
            for (int c = 0; c < m; c += 16) {   // cp[i]: the mass through item i
#pragma unroll
                for (int t = 0; t < 4; ++t) nx[t] = p4[min((c >> 2) + 4 + t, kSampleMaxK / 4 - 1)];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    float4 o;
                    pre += a[t].x; o.x = pre;
                    pre += a[t].y; o.y = pre;
                    pre += a[t].z; o.z = pre;
                    pre += a[t].w; o.w = pre;
                    cp4[(c >> 2) + t] = o;
                    a[t] = nx[t];
                }
            }
            int lim = m;   // cb[i] (the normalised mass before item i) is written for i < lim
            const float tp = prm->top_p;
            if (tp > 0.f && tp < 1.f && pre > 0.f) {
                const float inv = 1.0f / pre;
                float cum = 0.f;
#pragma unroll
                for (int t = 0; t < 4; ++t) a[t] = p4[t];
                for (int c = 0; c < m; c += 16) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) nx[t] = p4[min((c >> 2) + 4 + t, kSampleMaxK / 4 - 1)];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        float4 o;
                        o.x = cum; cum = __fadd_rn(cum, __fmul_rn(a[t].x, inv));
                        o.y = cum; cum = __fadd_rn(cum, __fmul_rn(a[t].y, inv));
                        o.z = cum; cum = __fadd_rn(cum, __fmul_rn(a[t].z, inv));
                        o.w = cum; cum = __fadd_rn(cum, __fmul_rn(a[t].w, inv));
                        cb4[(c >> 2) + t] = o;
                        a[t] = nx[t];
                    }
                    if (cum > tp) {   // the cut lies at or before item c + 16
                        lim = min(m, c + 16);
                        break;
                    }
                }
            } else {
                lim = 0;   // no cut
            }
            s_lim = lim;
        }
    }
    __syncthreads();
    if (wave == 0) {
        int tok = item_index(top[0]);
        float u = -1.f;
        if (draw) {
            // kept: the first item whose normalised mass before it exceeds top_p
            const int lim = s_lim;
            const float tp = prm->top_p;
            int kept = lim > 0 && lim < m ? lim : m;
            for (int c = 0; c < lim; c += 64) {
                const unsigned long long b = __ballot(c + lane < lim && cb[c + lane] > tp);
                if (b) {
                    kept = c + __ffsll((long long)b) - 1;
                    break;
                }
            }
            const uint64_t z = splitmix(prm->seed + (prm->counter + 1ull) * 0x9E3779B97F4A7C15ull);
            u = (float)(z >> 40) * 5.9604644775390625e-8f;   // [0, 1), 24 bits
            const float r = u * cp[kept - 1];   // u times the mass of the kept items
            // the first kept item whose running mass reaches r
            int d = 0;
            for (int c = 0; c < kept; c += 64) {
                const unsigned long long b = __ballot(c + lane < kept && cp[c + lane] >= r);
                if (b) {
                    d = c + __ffsll((long long)b) - 1;
                    break;
                }
            }
            tok = item_index(top[d]);
        }
        if (lane == 0) {
            if (draw) prm->counter += 1ull;
            out->u = u;
            out->token = tok;
            out->kept = m;
            if (win) {   // the step's input token onto the ring (the lists applied it)
                const int c = win->n, head = win->head;
                win->tok[c < kSampleWindow ? (head + c) % kSampleWindow : head] = st->token;
                win->head = c < kSampleWindow ? head : (head + 1) % kSampleWindow;
                win->n = c < kSampleWindow ? c + 1 : c;
            }
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
    // the decoder's window on the list path: the list kernel applies the
    // penalty and the select kernel pushes the token
    const bool fused_window = win && !large;
    if ((win && !fused_window) || (!win && recent && n_recent > 0)) {
        hipLaunchKernelGGL(k_penalty, dim3(1), dim3(kThreads), lds, st, logits, V,
                           win ? nullptr : recent, win ? 0 : n_recent, win, dstate, prm);
        TB_LAUNCHED();
    }
    if (large) {
        hipLaunchKernelGGL(k_topk_large, dim3(1), dim3(kLargeThreads), 0, st, logits, V, prm,
                           ws.key, ws.idx, ws.p, out, dstate, history, hist_cap);
        TB_LAUNCHED();
        return TB_OK;
    }
    uint64_t *lists = reinterpret_cast<uint64_t *>(ws.key);
    const int nbl = list_blocks(V);
    hipLaunchKernelGGL(k_topk_lists, dim3(nbl), dim3(kThreads), 0, st, logits, V, prm, lists,
                       ws.cnt, fused_window ? win : nullptr, dstate);
    TB_LAUNCHED();
    hipLaunchKernelGGL(k_topk_select, dim3(1), dim3(kSelThreads), 0, st, logits, V, nbl, lists,
                       ws.cnt, prm, out, dstate, history, hist_cap, fused_window ? win : nullptr);
    TB_LAUNCHED();
    return TB_OK;
}

}  // namespace tb

// The decoder handle: device-resident weights, KV cache and RoPE tables, and one
// captured hipGraph per token step.
//
// Replaces RustQwenDecoder (reference src/llm/decoder.rs:176-1374): `new`
// (193-424) -> tb_decoder_create / tb_decoder_set_layer, `step_internal`
// (1051-1374) -> the captured step, `decode_step` / `decode_and_sample` /
// `generate_loop` / `prefill_tokens` / `reset_kv_cache` /
// `copy_kv_cache_from_tensors` / `kv_len` / `get_logits` -> the tb_decoder_*
// entry points below.
//
// Step = embed -> L x [RMSNorm(+x records) -> QKV GEMV(+bias) -> RoPE + KV
// append -> split-KV attention (+x records) -> O GEMV (+residual) -> RMSNorm
// -> gate/up GEMV with silu*up -> x records of h -> down GEMV (+residual)] ->
// final RMSNorm -> lm_head GEMV -> device argmax.  Token and position live in a
// device state block, so the same graph replays for every step and a greedy
// generation runs without host round trips.
#include <limits.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <random>
#include <string>
#include <vector>

#include "../../include/tbhip_bench.h"
#include "decode.hpp"
#include "gemv_dense.hpp"
#include "tb_common.hpp"
#include "w4_gemv.hpp"
#include "w4_limb.hpp"
#include "w4_mfma.hpp"
#include "v2_layout.hpp"
#include "sample.hpp"

struct tb_decoder;

namespace tb {

namespace {

struct Layer {
    float *in_norm = nullptr, *post_norm = nullptr;
    void *qkv_w = nullptr, *o_w = nullptr, *gate_w = nullptr, *up_w = nullptr, *down_w = nullptr;
    float *qkv_s = nullptr, *o_s = nullptr, *gate_s = nullptr, *up_s = nullptr, *down_s = nullptr;
    float *qkv_b = nullptr;
    bool set = false;
};

int gshift(int64_t gs) { return gs == 32 ? 5 : 6; }
size_t up256(size_t b) { return (b + 255) & ~(size_t)255; }

}  // namespace

struct Decoder {
    tb_decoder_config cfg{};
    int H = 0, I = 0, hq = 0, hkv = 0, hd = 0, V = 0, L = 0, max_seq = 0, tq = 0, nsplit = 0;
    int wbits = 4, lmbits = 4, gs = 32;
    // Group 64 with every dimension a multiple of 64: the reference repacks QKV,
    // O, down and the lm_head into v2 blocks, so their scales are binary16
    // (decoder.rs:361-390); gate / up keep f32 scales.  Here those projections
    // keep v1 nibbles with scales rounded to binary16 at load: the same numbers
    // through the v1 GEMV, which streams faster than the 34-byte blocks.
    bool v2 = false;
    bool fused = true;   // RMSNorms fused into the GEMVs (TB_DECODER_UNFUSED=1: separate)
    // A step at position p attends positions 0 .. min(p + 1, attn_cap) - 1:
    // the native step's rule (decoder.rs:1179-1184) by default, INT_MAX for the
    // per-layer path's every-position attention (tb_decoder_set_attention_cap).
    int attn_cap = kNativeAttnCap;
    // W4A8 semantics (tb_set_vnni_semantics) at group 64: the mode the step
    // graphs were captured in (see enqueue_step_a8).
    bool a8 = false;
    // Rows per GEMV block for QKV, O, gate/up, down, lm_head (0 = the GEMV's
    // default; TB_DECODER_J="qkv,o,gu,down,lm" overrides, for tuning sweeps).
    int rj[5] = {0, 0, 0, 0, 0};
    float eps = 1e-6f;
    int device = 0;
    hipStream_t st = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    std::vector<void *> allocs;
    std::vector<Layer> layers;
    float *embed = nullptr, *final_norm = nullptr;
    void *lm_w = nullptr;
    float *lm_s = nullptr;
    float *kc = nullptr, *vc = nullptr, *cos_t = nullptr, *sin_t = nullptr;
    float *x = nullptr, *xn = nullptr, *qkv = nullptr, *attn = nullptr, *h = nullptr;
    float *logits = nullptr, *part = nullptr, *am_v = nullptr;
    float *xa = nullptr;   // W4A8: x' = q * s_x of the current projection input
    int *am_i = nullptr, *history = nullptr;
    uint32_t *xq_h = nullptr, *xq_a = nullptr, *xq_i = nullptr;
    float *ssq = nullptr;   // 16-element sums of squares of x (fused RMSNorm)
    DecState *state = nullptr;    // device
    DecState *hstate = nullptr;   // pinned host staging
    int hist_cap = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int64_t kv_used = 0;
    std::vector<float> host_logits;
    std::mt19937_64 rng{0x7B};   // host sampler (top_k beyond the device sampler's range)

    // Device sampler: parameters, result, candidates, the generation loop's
    // recent-token window, the decode_and_sample recent list, and the step
    // graph whose tail samples instead of taking the argmax.
    SampleParams *sprm = nullptr;
    SampleOut *sout = nullptr;
    SampleWindow *swin = nullptr;
    SampleScratch sws{};
    int64_t *srec = nullptr;
    int64_t srec_cap = 0;
    uint64_t seed = 0x7B, draws = 0;
    // sampled step graphs: [0] top_k <= kSampleMaxK (list / select path), [1] beyond
    hipGraph_t graph_s[2] = {nullptr, nullptr};
    hipGraphExec_t exec_s[2] = {nullptr, nullptr};
    bool tail_large = false;     // the sampler path enqueued by enqueue_tail
    bool sample_large = false;   // the path of the parameters set last

    ~Decoder() {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        for (int i = 0; i < 2; ++i) {
            if (exec_s[i]) (void)hipGraphExecDestroy(exec_s[i]);
            if (graph_s[i]) (void)hipGraphDestroy(graph_s[i]);
        }
        if (st) (void)hipStreamSynchronize(st);
        for (void *p : allocs) (void)hipFree(p);
        if (hstate) (void)hipHostFree(hstate);
        if (ev0) (void)hipEventDestroy(ev0);
        if (ev1) (void)hipEventDestroy(ev1);
        if (st) (void)hipStreamDestroy(st);
    }

    // Device memory.  Buffers under kArena / 4 are carved (256-byte aligned)
    // from arenas of kArena bytes, larger ones get their own allocation: the
    // decoder's hundreds of per-layer tensors then sit in a few large mappings
    // instead of one allocation each, whatever the process allocated before.
    static constexpr size_t kArena = (size_t)256 << 20;
    char *arena = nullptr;
    size_t arena_left = 0;

    int raw_alloc(void **q, size_t bytes) {
        hipError_t e = hipMalloc(q, bytes);
        if (e != hipSuccess)
            return fail(e == hipErrorOutOfMemory ? TB_ERR_MEMORY : TB_ERR_HIP,
                        "Out of memory allocating " + std::to_string(bytes >> 20) +
                            " MB for the decoder on the GPU: " + hipGetErrorString(e));
        allocs.push_back(*q);
        return TB_OK;
    }

    template <class T>
    int alloc(T **p, size_t bytes) {
        bytes = (bytes + 255) & ~(size_t)255;
        if (bytes == 0) bytes = 256;
        void *q = nullptr;
        int rc;
        if (bytes >= kArena / 4) {
            if ((rc = raw_alloc(&q, bytes))) return rc;
        } else {
            if (bytes > arena_left) {
                void *a = nullptr;
                if ((rc = raw_alloc(&a, kArena))) return rc;
                arena = static_cast<char *>(a);
                arena_left = kArena;
            }
            q = arena;
            arena += bytes;
            arena_left -= bytes;
        }
        *p = static_cast<T *>(q);
        return TB_OK;
    }

    // Device copy of a caller buffer (host or device memory).
    template <class T>
    int upload(T **dst, const void *src, size_t bytes) {
        int rc = alloc(dst, bytes);
        if (rc) return rc;
        TB_HIP(hipMemcpy(*dst, src, bytes, hipMemcpyDefault));
        return TB_OK;
    }

    // An INT4 projection [n, k] whose scales the reference holds in binary16
    // (v2 repack, group 64): v1 nibbles as given, scales rounded to binary16
    // on the device (f32_to_f16, packed_v2.rs:66-105).
    int upload_f16_scaled(void **w_dst, float **s_dst, const void *w, const float *s, int64_t n,
                          int64_t k) {
        int rc;
        if ((rc = upload(w_dst, w, wbytes(4, n, k))) || (rc = upload(s_dst, s, sbytes(4, n, k))))
            return rc;
        if ((rc = round_scales_f16(*s_dst, n * (k / gs), st))) return rc;
        TB_HIP(hipStreamSynchronize(st));
        return TB_OK;
    }

    size_t wbytes(int bits, int64_t n, int64_t k) const {
        return bits == 4 ? (size_t)n * (size_t)((k + 1) / 2)
                         : (size_t)n * (size_t)k * (bits == 8 ? 1 : 4);
    }
    size_t sbytes(int bits, int64_t n, int64_t k) const {
        return bits == 4 ? (size_t)n * (size_t)(k / gs) * 4 : (bits == 8 ? (size_t)n * 4 : 0);
    }

    // Fused-RMSNorm wiring of a projection: the input side (sums of squares of
    // x; x * w_norm as records for INT4, in f32 for INT8 / fp32) and the output
    // side (y * rec_w as records (INT4 only) and in f32, and the 16-row sums of
    // squares of y).
    struct Fuse {
        const float *ssq_in = nullptr;
        uint32_t *rec_out = nullptr;
        const float *rec_w = nullptr;
        float *xw_out = nullptr;
        float *ssq_out = nullptr;
    };

    // One projection y = W x [+ bias] [+ residual] or the gate/up pair.
    int proj(int bits, const float *xin, const uint32_t *xq, const void *w, const float *s,
             const float *b, const void *w2, const float *s2, const float *res, float *y,
             int n, int k, int epi, const RopeArgs *rope = nullptr, const Fuse *fu = nullptr,
             int rows_j = 0) {
        if (bits == 4) {
            W4Params p{};
            p.rows_j = rows_j;
            p.x = xin; p.xq = xq;
            p.w0 = static_cast<const uint8_t *>(w); p.s0 = s; p.b0 = b;
            p.w1 = static_cast<const uint8_t *>(w2); p.s1 = s2;
            p.res = res; p.y = y; p.m = 1; p.n = n; p.k = k; p.gshift = gshift(gs);
            if (rope) p.rope = *rope;
            if (fu) {
                p.ssq_in = fu->ssq_in;
                p.ssq_n = H / 16;
                p.norm_h = H;
                p.eps = eps;
                p.rec_out = fu->rec_out;
                p.rec_w = fu->rec_w;
                p.xw_out = fu->xw_out;
                p.ssq_out = fu->ssq_out;
            }
            return w4_gemv(p, epi, st);
        }
        DenseParams p{};
        p.x = xin; p.w0 = w; p.rs0 = s; p.rs0_len = s ? n : 0; p.b0 = b;
        p.w1 = w2; p.rs1 = s2; p.rs1_len = s2 ? n : 0;
        p.res = res; p.y = y; p.m = 1; p.n = n; p.k = k;
        if (rope) p.rope = *rope;
        if (fu) {
            p.ssq_in = fu->ssq_in;
            p.ssq_n = H / 16;
            p.norm_h = H;
            p.eps = eps;
            p.rec_w = fu->rec_w;
            p.xw_out = fu->xw_out;
            p.ssq_out = fu->ssq_out;
        }
        return dense_gemv(p, bits == 8 ? W_I8 : W_F32, epi, st);
    }

    // The step with every RMSNorm fused into the GEMVs around it: the
    // producer of x (embedding, O and down projections) writes x * w_norm in
    // f32 to xn (INT4: also its records; the f32 copy is then read only on the
    // NaN/Inf path) and the 16-element sums of squares of x; the consumer
    // (QKV, gate/up, lm_head) scales its dots by 1 / rms.  INT4: h's records
    // come from the gate/up epilogue.  Kernels per layer: QKV, attention
    // (split + merge), O, gate/up, down.
    // The step's tail: greedy argmax, or the device sampler over the window.
    int enqueue_tail(bool sampled) {
        if (!sampled) return launch_argmax(logits, V, am_v, am_i, state, history, hist_cap, st);
        return launch_sample(logits, V, nullptr, 0, sprm, sws, sout, st, tail_large, swin, state,
                             history, hist_cap);
    }

    int enqueue_step_fused(bool sampled) {
        const int wb = wbits;
        const bool q4 = wb == 4;
        int rc = launch_embed_rec(state, embed, x, layers[0].in_norm, xn, xq_h, ssq, H, st);
        if (rc) return rc;
        for (int l = 0; l < L; ++l) {
            const Layer &y = layers[l];
            float *kcl = kc + (size_t)l * hkv * max_seq * hd;
            float *vcl = vc + (size_t)l * hkv * max_seq * hd;
            RopeArgs ra{&state->pos, cos_t, sin_t, kcl, vcl, hq, hkv, hd, max_seq, hd};
            Fuse fq;
            fq.ssq_in = ssq;
            rc = proj(wb, xn, xq_h, y.qkv_w, y.qkv_s, y.qkv_b, nullptr, nullptr, nullptr, qkv, tq,
                      H, EPI_ROPE, &ra, &fq, rj[0]);
            if (rc) return rc;
            rc = launch_attention(state, qkv, kcl, vcl, part, attn, q4 ? xq_a : nullptr, hq, hkv,
                                  hd, max_seq, attn_cap, st);
            if (rc) return rc;
            Fuse fo;
            fo.rec_out = q4 ? xq_h : nullptr;
            fo.rec_w = y.post_norm;
            fo.xw_out = xn;
            fo.ssq_out = ssq;
            rc = proj(wb, attn, xq_a, y.o_w, y.o_s, nullptr, nullptr, nullptr, x, x, H, hq * hd,
                      EPI_RESID, nullptr, &fo, rj[1]);
            if (rc) return rc;
            Fuse fg;
            fg.ssq_in = ssq;
            fg.rec_out = q4 ? xq_i : nullptr;
            rc = proj(wb, xn, xq_h, y.gate_w, y.gate_s, nullptr, y.up_w, y.up_s, nullptr, h, I, H,
                      EPI_SWIGLU, nullptr, &fg, rj[2]);
            if (rc) return rc;
            Fuse fd;
            fd.rec_out = q4 ? xq_h : nullptr;
            fd.rec_w = l + 1 < L ? layers[l + 1].in_norm : final_norm;
            fd.xw_out = xn;
            fd.ssq_out = ssq;
            rc = proj(wb, h, xq_i, y.down_w, y.down_s, nullptr, nullptr, nullptr, x, x, H, I,
                      EPI_RESID, nullptr, &fd, rj[3]);
            if (rc) return rc;
        }
        // lm_head: INT4, INT8 or fp32, always a fused-RMSNorm consumer of xn.
        Fuse fl;
        fl.ssq_in = ssq;
        rc = proj(lmbits, xn, xq_h, lm_w, lm_s, nullptr, nullptr, nullptr, nullptr, logits, V, H,
                  EPI_PLAIN, nullptr, &fl, rj[4]);
        if (rc) return rc;
        return enqueue_tail(sampled);
    }

    // The step under W4A8 semantics at group 64 (tb_set_vnni_semantics).  On
    // an AVX-512 VNNI host the reference rounds the input of every group-64
    // INT4 projection to bytes: the SwiGLU pair's (decoder.rs:1262-1282) and,
    // through projection_gemv (decoder.rs:1029-1049 -> packed_v2.rs:366-370 or
    // gemv.rs:1559-1563), QKV's, O's, down's and the INT4 lm_head's.  The
    // RMSNorms run as separate kernels (the rounding takes the maximum of the
    // normalised row), and one pass per projection input writes x' = q * s_x
    // and its records.  The weights are those of the exact step (binary16
    // scales where the reference repacks to v2 blocks).
    bool a8_wanted() const { return wbits == 4 && gs == 64 && vnni_semantics(); }

    int enqueue_step_a8(bool sampled) {
        int rc;
        const int qd = hq * hd;
        for (int l = 0; l < L; ++l) {
            const Layer &y = layers[l];
            float *kcl = kc + (size_t)l * hkv * max_seq * hd;
            float *vcl = vc + (size_t)l * hkv * max_seq * hd;
            RopeArgs ra{&state->pos, cos_t, sin_t, kcl, vcl, hq, hkv, hd, max_seq, hd};
            if ((rc = launch_rmsnorm(state, l == 0 ? embed : nullptr, x, y.in_norm, xn, nullptr, H,
                                     eps, st)) ||
                (rc = act_rec(xn, xa, xq_h, 1, H, st)) ||
                (rc = proj(4, xa, xq_h, y.qkv_w, y.qkv_s, y.qkv_b, nullptr, nullptr, nullptr, qkv,
                           tq, H, EPI_ROPE, &ra)) ||
                (rc = launch_attention(state, qkv, kcl, vcl, part, attn, nullptr, hq, hkv, hd,
                                       max_seq, attn_cap, st)) ||
                (rc = act_rec(attn, xa, xq_a, 1, qd, st)) ||
                (rc = proj(4, xa, xq_a, y.o_w, y.o_s, nullptr, nullptr, nullptr, x, x, H, qd,
                           EPI_RESID)) ||
                (rc = launch_rmsnorm(state, nullptr, x, y.post_norm, xn, nullptr, H, eps, st)) ||
                (rc = act_rec(xn, xa, xq_h, 1, H, st)) ||
                (rc = proj(4, xa, xq_h, y.gate_w, y.gate_s, nullptr, y.up_w, y.up_s, nullptr, h,
                           I, H, EPI_SWIGLU)) ||
                (rc = act_rec(h, xa, xq_i, 1, I, st)) ||
                (rc = proj(4, xa, xq_i, y.down_w, y.down_s, nullptr, nullptr, nullptr, x, x, H, I,
                           EPI_RESID)))
                return rc;
        }
        if ((rc = launch_rmsnorm(state, nullptr, x, final_norm, xn, nullptr, H, eps, st))) return rc;
        const float *lin = xn;
        const uint32_t *lq = nullptr;
        if (lmbits == 4) {
            if ((rc = act_rec(xn, xa, xq_h, 1, H, st))) return rc;
            lin = xa;
            lq = xq_h;
        }
        if ((rc = proj(lmbits, lin, lq, lm_w, lm_s, nullptr, nullptr, nullptr, nullptr, logits, V,
                       H, EPI_PLAIN)))
            return rc;
        return enqueue_tail(sampled);
    }

    // Enqueues one decoder step (reference step_internal) on `st`.
    int enqueue_step(bool sampled = false) {
        if (a8) return enqueue_step_a8(sampled);
        const bool q4 = wbits == 4;
        // INT8 layers write no records, which an INT4 lm_head reads: that pair
        // keeps the separate final RMSNorm of the unfused step.
        if (fused && (wbits == 4 || lmbits != 4)) return enqueue_step_fused(sampled);
        int rc;
        for (int l = 0; l < L; ++l) {
            const Layer &y = layers[l];
            float *kcl = kc + (size_t)l * hkv * max_seq * hd;
            float *vcl = vc + (size_t)l * hkv * max_seq * hd;
            rc = launch_rmsnorm(state, l == 0 ? embed : nullptr, x, y.in_norm, xn,
                                q4 ? xq_h : nullptr, H, eps, st);
            if (rc) return rc;
            // QKV projection + bias + RoPE + KV-cache append in one kernel.
            RopeArgs ra{&state->pos, cos_t, sin_t, kcl, vcl, hq, hkv, hd, max_seq, hd};
            rc = proj(wbits, xn, xq_h, y.qkv_w, y.qkv_s, y.qkv_b, nullptr, nullptr, nullptr, qkv,
                      tq, H, EPI_ROPE, &ra);
            if (rc) return rc;
            rc = launch_attention(state, qkv, kcl, vcl, part, attn, q4 ? xq_a : nullptr, hq, hkv,
                                  hd, max_seq, attn_cap, st);
            if (rc) return rc;
            rc = proj(wbits, attn, xq_a, y.o_w, y.o_s, nullptr, nullptr, nullptr, x, x, H,
                      hq * hd, EPI_RESID);
            if (rc) return rc;
            rc = launch_rmsnorm(state, nullptr, x, y.post_norm, xn, q4 ? xq_h : nullptr, H, eps,
                                st);
            if (rc) return rc;
            rc = proj(wbits, xn, xq_h, y.gate_w, y.gate_s, nullptr, y.up_w, y.up_s, nullptr, h, I,
                      H, EPI_SWIGLU);
            if (rc) return rc;
            if (q4) {
                rc = xquant(h, xq_i, 1, I, st);
                if (rc) return rc;
            }
            rc = proj(wbits, h, xq_i, y.down_w, y.down_s, nullptr, nullptr, nullptr, x, x, H, I,
                      EPI_RESID);
            if (rc) return rc;
        }
        rc = launch_rmsnorm(state, nullptr, x, final_norm, xn, lmbits == 4 ? xq_h : nullptr, H,
                            eps, st);
        if (rc) return rc;
        rc = proj(lmbits, xn, xq_h, lm_w, lm_s, nullptr, nullptr, nullptr, nullptr, logits, V, H,
                  EPI_PLAIN);
        if (rc) return rc;
        return enqueue_tail(sampled);
    }

    int capture(bool sampled, hipGraph_t *gr, hipGraphExec_t *ex) {
        for (int l = 0; l < L; ++l)
            TB_REQUIRE(layers[l].set, TB_ERR_VALUE,
                       "decoder layer " + std::to_string(l) + " was never set");
        TB_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        int rc = enqueue_step(sampled);
        hipGraph_t g = nullptr;
        hipError_t e = hipStreamEndCapture(st, &g);
        if (rc) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess) return fail(TB_ERR_HIP, std::string("graph capture: ") + hipGetErrorString(e));
        *gr = g;
        TB_HIP(hipGraphInstantiate(ex, g, nullptr, nullptr, 0));
        return TB_OK;
    }

    // The step graphs follow the W4A8 switch: a change drops them.
    int sync_a8() {
        const bool want = a8_wanted();
        if (want == a8) return TB_OK;
        TB_HIP(hipStreamSynchronize(st));
        int rc = drop_graphs();
        if (rc) return rc;
        a8 = want;
        return TB_OK;
    }

    int ensure_graph() {
        int rc = sync_a8();
        if (rc) return rc;
        return exec ? TB_OK : capture(false, &graph, &exec);
    }

    // Destroys the captured step graphs; the next step captures them again.
    int drop_graphs() {
        if (exec) TB_HIP(hipGraphExecDestroy(exec));
        if (graph) TB_HIP(hipGraphDestroy(graph));
        for (int i = 0; i < 2; ++i) {
            if (exec_s[i]) TB_HIP(hipGraphExecDestroy(exec_s[i]));
            if (graph_s[i]) TB_HIP(hipGraphDestroy(graph_s[i]));
            exec_s[i] = nullptr;
            graph_s[i] = nullptr;
        }
        exec = nullptr;
        graph = nullptr;
        return TB_OK;
    }

    // ---- Device sampling -----------------------------------------------------
    int sampler_alloc() {
        if (sprm) return TB_OK;
        int rc;
        if ((rc = alloc(&sprm, sizeof(SampleParams))) || (rc = alloc(&sout, sizeof(SampleOut))) ||
            (rc = alloc(&swin, sizeof(SampleWindow))) ||
            (rc = alloc(&sws.key, (size_t)sample_scratch_items(V) * 4)) ||
            (rc = alloc(&sws.idx, (size_t)sample_scratch_items(V) * 4)) ||
            (rc = alloc(&sws.p, (size_t)sample_scratch_items(V) * 4)) ||
            (rc = alloc(&sws.cnt, (size_t)kSampleLists * 4)))
            return rc;
        return TB_OK;
    }

    // The sampled step graph of the path the parameters set last call for.
    int ensure_graph_s() {
        int rc = sampler_alloc();
        if (rc || (rc = sync_a8())) return rc;
        const int i = sample_large ? 1 : 0;
        if (exec_s[i]) return TB_OK;
        tail_large = sample_large;
        return capture(true, &graph_s[i], &exec_s[i]);
    }
    hipGraphExec_t sampled_graph() const { return exec_s[sample_large ? 1 : 0]; }

    // Upload of the sampling parameters (the draw counter continues the stream).
    int set_sampler(float temperature, int64_t top_k, float top_p, float penalty) {
        int rc = sampler_alloc();
        if (rc) return rc;
        const bool greedy = !std::isfinite(temperature) || temperature <= 0.f || top_k == 1;
        SampleParams p{};
        p.temperature = temperature;
        p.top_p = top_p;
        p.penalty = penalty;
        p.k = greedy ? 1 : (int)std::max<int64_t>(1, std::min<int64_t>(top_k, V));
        p.greedy = greedy ? 1 : 0;
        p.seed = seed;
        p.counter = draws;
        sample_large = p.k > kSampleMaxK;
        TB_HIP(hipMemcpyAsync(sprm, &p, sizeof(p), hipMemcpyHostToDevice, st));
        return TB_OK;
    }

    // The draw counter after device draws, and the drawn token.
    int sampler_result(int64_t *token) {
        SampleParams p{};
        SampleOut o{};
        TB_HIP(hipMemcpyAsync(&p, sprm, sizeof(p), hipMemcpyDeviceToHost, st));
        TB_HIP(hipMemcpyAsync(&o, sout, sizeof(o), hipMemcpyDeviceToHost, st));
        TB_HIP(hipStreamSynchronize(st));
        draws = p.counter;
        if (token) *token = o.token;
        return TB_OK;
    }

    // Every top_k samples on the device (top_k > kSampleMaxK on the one-block
    // path); the host sampler remains for vocabularies past 262144 tokens.
    bool device_samplable(float, int64_t) const { return V <= kSampleMaxBlocks * kSampleSlice; }

    // decode_and_sample on the device: one step, then the sampler over the
    // logits with the caller's recent tokens.
    int step_and_sample(int64_t token, int64_t pos, float temperature, int64_t top_k, float top_p,
                        float penalty, const int64_t *recent, int64_t n_recent, int64_t *out) {
        int rc = step(token, pos, false, nullptr);
        if (rc) return rc;
        if ((rc = set_sampler(temperature, top_k, top_p, penalty))) return rc;
        if (penalty > 1.0f && n_recent > 0) {
            if (n_recent > srec_cap) {
                if ((rc = alloc(&srec, (size_t)n_recent * 8))) return rc;
                srec_cap = n_recent;
            }
            TB_HIP(hipMemcpyAsync(srec, recent, (size_t)n_recent * 8, hipMemcpyHostToDevice, st));
        }
        if ((rc = launch_sample(logits, V, srec, penalty > 1.0f ? (int)n_recent : 0, sprm, sws,
                                sout, st, sample_large)))
            return rc;
        return sampler_result(out);
    }

    int set_state(int token, int pos) {
        hstate->token = token;
        hstate->pos = pos;
        hstate->step = 0;
        hstate->argmax = 0;
        TB_HIP(hipMemcpyAsync(state, hstate, sizeof(DecState), hipMemcpyHostToDevice, st));
        return TB_OK;
    }

    // ---- Batched prefill (INT4 projections on the FP32-MFMA GEMM) ----------
    // Chunks of up to kPrefillRows prompt positions go through each layer as
    // one batch: row RMSNorms, QKV GEMM (+bias), RoPE + KV append for every
    // row, causal prefill attention, O GEMM + residual, gate/up GEMM with
    // SwiGLU, down GEMM + residual; the last row then takes the final norm
    // and lm_head as a step would.  Buffers are allocated on first use.
    static constexpr int kPrefillRows = 256;
    float *pf_x = nullptr, *pf_xn = nullptr, *pf_qkv = nullptr, *pf_q = nullptr,
          *pf_a = nullptr, *pf_h = nullptr, *pf_part = nullptr;
    int *pf_tok = nullptr;

    int prefill_alloc() {
        if (pf_x) return TB_OK;
        const int R = kPrefillRows;
        const size_t nq = (size_t)(hq + 2 * hkv) * hd;
        size_t part = w4_mfma_partials_bytes(R, (int)nq, H, false);
        part = std::max(part, w4_mfma_partials_bytes(R, H, hq * hd, false));
        part = std::max(part, w4_mfma_partials_bytes(R, I, H, true));
        part = std::max(part, w4_mfma_partials_bytes(R, H, I, false));
        // 3..16 rows (verify_tokens, short chunks) take the small-batch
        // projection: records + split partials of the largest of its shapes
        size_t lb = 0;
        for (int m = 3; m <= kLimbMaxM; ++m) {
            auto need = [&](int n, int k, bool pair) -> size_t {
                if (!limb_shape_ok(m, n, k, pair)) return 0;
                return up256(limb_records_bytes(m, k)) + limb_partials_bytes(m, n, k, pair);
            };
            lb = std::max({lb, need((int)nq, H, false), need(H, hq * hd, false), need(I, H, true),
                           need(H, I, false)});
            if (m <= 8 && lmbits == 4) lb = std::max(lb, need(V, H, false));
        }
        int rc;
        if ((rc = alloc(&pf_x, (size_t)R * H * 4)) || (rc = alloc(&pf_xn, (size_t)R * H * 4)) ||
            (rc = alloc(&pf_qkv, (size_t)R * nq * 4)) ||
            (rc = alloc(&pf_q, (size_t)R * hq * hd * 4)) ||
            (rc = alloc(&pf_a, (size_t)R * hq * hd * 4)) || (rc = alloc(&pf_h, (size_t)R * I * 4)) ||
            (rc = alloc(&pf_part, part)) || (rc = alloc(&pf_tok, (size_t)R * 4)) ||
            (lb && (rc = alloc(&pf_limb, lb))) ||
            (lb && (rc = alloc(&pf_hrec, limb_records_bytes(kLimbMaxM, I)))))
            return rc;
        pf_limb_bytes = lb;
        return TB_OK;
    }

    // The small-batch projection (records of x, then w4_limb) when it takes
    // the shape and the buffer holds its scratch; false: use the GEMM.
    // rec_out (a SwiGLU pair): the pair also writes the records of h there;
    // rec_in: records of xin already built (by such a pair), no record pass.
    uint8_t *pf_limb = nullptr;
    uint8_t *pf_hrec = nullptr;   // records of h, [kLimbMaxM, I]
    size_t pf_limb_bytes = 0;
    bool limb_gemm(const float *xin, const void *w, const float *s, const float *b,
                   const void *w2, const float *s2, const float *res, float *y, int m, int n,
                   int k, int &rc, uint8_t *rec_out = nullptr, const uint8_t *rec_in = nullptr) {
        const bool pair = w2 != nullptr;
        if (!pf_limb || m < 3 || m > kLimbMaxM || !limb_shape_ok(m, n, k, pair)) return false;
        const size_t rb = up256(limb_records_bytes(m, k));
        if (rb + limb_partials_bytes(m, n, k, pair) > pf_limb_bytes) return false;
        LimbParams p{};
        p.x = xin; p.rec = rec_in ? rec_in : pf_limb;
        p.w0 = static_cast<const uint8_t *>(w); p.s0 = s; p.b0 = b;
        p.w1 = static_cast<const uint8_t *>(w2); p.s1 = s2;
        p.res = res; p.y = y; p.m = m; p.n = n; p.k = k;
        p.scols = k / gs; p.gshift = gshift(gs);
        p.rec_out = pair ? rec_out : nullptr;
        if (!rec_in && (rc = limb_prep(xin, pf_limb, m, k, st))) return true;
        rc = w4_limb(p, reinterpret_cast<float *>(pf_limb + rb), st);
        return true;
    }

    // The SwiGLU pair then the down projection (+ residual): on the
    // small-batch path the pair writes h's records and the down projection
    // reads them (no record pass for h).
    int mlp_rows(const Layer &y, int M) {
        int rc = TB_OK;
        if (pf_hrec && limb_gemm(pf_xn, y.gate_w, y.gate_s, nullptr, y.up_w, y.up_s, nullptr,
                                 pf_h, M, I, H, rc, pf_hrec)) {
            if (rc) return rc;
            if (limb_gemm(pf_h, y.down_w, y.down_s, nullptr, nullptr, nullptr, pf_x, pf_x, M, H,
                          I, rc, nullptr, pf_hrec))
                return rc;
            return gemm(pf_h, y.down_w, y.down_s, nullptr, nullptr, nullptr, pf_x, pf_x, M, H, I,
                        EPI_RESID);
        }
        if ((rc = gemm(pf_xn, y.gate_w, y.gate_s, nullptr, y.up_w, y.up_s, nullptr, pf_h, M, I,
                       H, EPI_SWIGLU)))
            return rc;
        return gemm(pf_h, y.down_w, y.down_s, nullptr, nullptr, nullptr, pf_x, pf_x, M, H, I,
                    EPI_RESID);
    }

    int gemm(const float *xin, const void *w, const float *s, const float *b, const void *w2,
             const float *s2, const float *res, float *y, int m, int n, int k, int epi) {
        int rc = TB_OK;
        if (limb_gemm(xin, w, s, b, w2, s2, res, y, m, n, k, rc)) return rc;
        MfmaParams p{};
        p.x = xin;
        p.w0 = static_cast<const uint8_t *>(w); p.s0 = s; p.b0 = b;
        p.w1 = static_cast<const uint8_t *>(w2); p.s1 = s2;
        p.res = res; p.y = y; p.m = m; p.n = n; p.k = k; p.gshift = gshift(gs);
        return w4_mfma(p, epi, pf_part, st);
    }

    // Positions start .. start + n - 1 attend every earlier position (the
    // batched attention has no cap), so chunks reaching the cap take the step
    // loop.
    bool under_cap(int64_t start, int64_t n) const { return start + n <= (int64_t)attn_cap; }

    bool prefill_batchable(const int64_t *tokens, int64_t n, int64_t start) const {
        static const bool loop_only = getenv("TB_PREFILL_LOOP") != nullptr;
        // W4A8 rounds each token's projection inputs: the step loop does that
        if (loop_only || wbits != 4 || n < 16 || !under_cap(start, n) || a8_wanted()) return false;
        for (int64_t i = 0; i < n; ++i)
            if (tokens[i] < 0 || tokens[i] >= V) return false;   // the step's zero-logit rule
        return true;
    }

    // The lm_head over M rows of normalised hidden states xr [M, H] into
    // y [M, V]: the MFMA GEMM for INT4 (64 rows per launch, its split-K
    // partials in pf_lmpart), GEMV passes of 2 rows for INT8 / fp32.
    float *pf_lmpart = nullptr;
    float *pf_attn = nullptr;    // key-range split partials of the prefill attention
    size_t pf_attn_bytes = 0;
    float *pf_rows = nullptr;    // verify_tokens: logits of every position
    int64_t pf_rows_n = 0;
    int lm_rows(const float *xr, float *y, int M) {
        int rc;
        if (lmbits == 4) {
            if (M <= 8 && limb_gemm(xr, lm_w, lm_s, nullptr, nullptr, nullptr, nullptr, y, M, V, H,
                                    rc))
                return rc;
            if (!pf_lmpart &&
                (rc = alloc(&pf_lmpart, w4_mfma_partials_bytes(64, V, H, false))))
                return rc;
            for (int r0 = 0; r0 < M; r0 += 64) {
                MfmaParams p{};
                p.x = xr + (size_t)r0 * H;
                p.w0 = static_cast<const uint8_t *>(lm_w); p.s0 = lm_s;
                p.y = y + (size_t)r0 * V; p.m = std::min(64, M - r0); p.n = V; p.k = H;
                p.gshift = gshift(gs);
                if ((rc = w4_mfma(p, EPI_PLAIN, pf_lmpart, st))) return rc;
            }
            return TB_OK;
        }
        for (int r0 = 0; r0 < M; r0 += 2) {
            DenseParams p{};
            p.x = xr + (size_t)r0 * H; p.w0 = lm_w; p.rs0 = lm_s; p.rs0_len = lm_s ? V : 0;
            p.y = y + (size_t)r0 * V; p.m = std::min(2, M - r0); p.n = V; p.k = H;
            if ((rc = dense_gemv(p, lmbits == 8 ? W_I8 : W_F32, EPI_PLAIN, st))) return rc;
        }
        return TB_OK;
    }

    // rows_out (device [n, V]): every position's logits, as verify_tokens
    // returns them (decoder.rs:565-581); otherwise only the last position's.
    int prefill_batched(const int64_t *tokens, int64_t n, int64_t start,
                        float *rows_out = nullptr) {
        int rc = prefill_alloc();
        if (rc) return rc;
        const int nq = (hq + 2 * hkv) * hd;
        // Host copy of the whole prompt, alive until the closing synchronize.
        std::vector<int> tok32(tokens, tokens + n);
        for (int64_t c0 = 0; c0 < n; c0 += kPrefillRows) {
            const int M = (int)std::min<int64_t>(kPrefillRows, n - c0);
            const int pos0 = (int)(start + c0);
            TB_HIP(hipMemcpyAsync(pf_tok, tok32.data() + c0, (size_t)M * 4, hipMemcpyHostToDevice,
                                  st));
            const size_t ab = prefill_attention_scratch(
                M, hq, hd, prefill_attention_splits(pos0, M, hq, hkv));
            if (ab > pf_attn_bytes) {
                if ((rc = alloc(&pf_attn, ab))) return rc;
                pf_attn_bytes = ab;
            }
            if ((rc = launch_embed_rows(pf_tok, embed, pf_x, M, H, st))) return rc;
            for (int l = 0; l < L; ++l) {
                const Layer &y = layers[l];
                float *kcl = kc + (size_t)l * hkv * max_seq * hd;
                float *vcl = vc + (size_t)l * hkv * max_seq * hd;
                if ((rc = launch_rmsnorm_rows(pf_x, y.in_norm, pf_xn, M, H, eps, st)) ||
                    (rc = gemm(pf_xn, y.qkv_w, y.qkv_s, y.qkv_b, nullptr, nullptr, nullptr, pf_qkv,
                               M, nq, H, EPI_PLAIN)) ||
                    (rc = launch_rope_rows(pf_qkv, pf_q, kcl, vcl, cos_t, sin_t, pos0, M, hq, hkv,
                                           hd, max_seq, st)) ||
                    (rc = launch_prefill_attention(pf_q, kcl, vcl, pf_a, pos0, M, hq, hkv, hd,
                                                   max_seq, pf_attn, st)) ||
                    (rc = gemm(pf_a, y.o_w, y.o_s, nullptr, nullptr, nullptr, pf_x, pf_x, M, H,
                               hq * hd, EPI_RESID)) ||
                    (rc = launch_rmsnorm_rows(pf_x, y.post_norm, pf_xn, M, H, eps, st)) ||
                    (rc = mlp_rows(y, M)))
                    return rc;
            }
            if (rows_out) {
                if ((rc = launch_rmsnorm_rows(pf_x, final_norm, pf_xn, M, H, eps, st)) ||
                    (rc = lm_rows(pf_xn, rows_out + (size_t)c0 * V, M)))
                    return rc;
                if (c0 + M == n)
                    TB_HIP(hipMemcpyAsync(logits, rows_out + (size_t)(n - 1) * V, (size_t)V * 4,
                                          hipMemcpyDeviceToDevice, st));
            } else if (c0 + M == n) {
                // The last position's hidden state -> final norm -> lm_head.
                TB_HIP(hipMemcpyAsync(x, pf_x + (size_t)(M - 1) * H, (size_t)H * 4,
                                      hipMemcpyDeviceToDevice, st));
                if ((rc = launch_rmsnorm(state, nullptr, x, final_norm, xn,
                                         lmbits == 4 ? xq_h : nullptr, H, eps, st)) ||
                    (rc = proj(lmbits, xn, xq_h, lm_w, lm_s, nullptr, nullptr, nullptr, nullptr,
                               logits, V, H, EPI_PLAIN)))
                    return rc;
            }
        }
        kv_used = std::max<int64_t>(kv_used, start + n);
        TB_HIP(hipMemcpyAsync(host_logits.data(), logits, (size_t)V * 4, hipMemcpyDeviceToHost, st));
        TB_HIP(hipStreamSynchronize(st));
        return TB_OK;
    }

    bool in_range(int64_t token, int64_t pos) const {
        return token >= 0 && token < V && pos >= 0 && pos < max_seq;
    }

    // One step; out-of-range token or position gives zero logits and touches
    // nothing else (decoder.rs:1066-1089).
    int step(int64_t token, int64_t pos, bool want_logits, int64_t *argmax) {
        int rc = ensure_graph();
        if (rc) return rc;
        if (!in_range(token, pos)) {
            TB_HIP(hipMemsetAsync(logits, 0, (size_t)V * 4, st));
            TB_HIP(hipStreamSynchronize(st));
            if (want_logits) std::fill(host_logits.begin(), host_logits.end(), 0.f);
            if (argmax) *argmax = 0;
            return TB_OK;
        }
        kv_used = std::max<int64_t>(kv_used, pos + 1);
        rc = set_state((int)token, (int)pos);
        if (rc) return rc;
        TB_HIP(hipGraphLaunch(exec, st));
        if (want_logits)
            TB_HIP(hipMemcpyAsync(host_logits.data(), logits, (size_t)V * 4, hipMemcpyDeviceToHost,
                                  st));
        if (argmax) TB_HIP(hipMemcpyAsync(hstate, state, sizeof(DecState), hipMemcpyDeviceToHost, st));
        TB_HIP(hipStreamSynchronize(st));
        if (argmax) *argmax = hstate->argmax;
        return TB_OK;
    }
};

// Repetition penalty (src/llm/decoder.rs:878-899): each distinct recent token's
// logit is divided by the penalty when positive, multiplied when not.
static void repetition_penalty(std::vector<float> &lg, const int64_t *recent, int64_t n,
                               float penalty) {
    if (penalty <= 1.0f || n <= 0) return;
    std::vector<int64_t> seen;
    for (int64_t i = 0; i < n; ++i) {
        const int64_t t = recent[i];
        if (t < 0 || t >= (int64_t)lg.size()) continue;
        if (std::find(seen.begin(), seen.end(), t) != seen.end()) continue;
        seen.push_back(t);
        const float l = lg[t];
        lg[t] = l > 0.f ? l / penalty : l * penalty;
    }
}

// Sampling of src/llm/decoder.rs:908-1020: greedy (strict >, lowest index) when
// temperature is not finite or <= 0 or top_k == 1; otherwise the top-k
// candidates (non-finite logits as -inf), softmax at `temperature`, optional
// nucleus cut at top_p, then one multinomial draw.  The reference draws from
// rand::random (unseeded); this draws from the decoder's seeded generator.
static int64_t sample(const std::vector<float> &lg, float temperature, int64_t top_k, float top_p,
                      std::mt19937_64 &rng) {
    const int64_t V = (int64_t)lg.size();
    if (V == 0) return 0;
    if (!std::isfinite(temperature) || temperature <= 0.f || top_k == 1) {
        int64_t bi = 0;
        float bv = lg[0];
        for (int64_t i = 1; i < V; ++i)
            if (lg[i] > bv) {
                bv = lg[i];
                bi = i;
            }
        return bi;
    }
    const int64_t k = std::max<int64_t>(1, std::min<int64_t>(top_k, V));
    std::vector<std::pair<int64_t, float>> items((size_t)V);
    for (int64_t i = 0; i < V; ++i) items[i] = {i, std::isfinite(lg[i]) ? lg[i] : -INFINITY};
    std::partial_sort(items.begin(), items.begin() + k, items.end(),
                      [](const auto &a, const auto &b) { return a.second > b.second; });
    items.resize((size_t)k);
    const float mx = items[0].second;
    const float inv_t = 1.0f / temperature;
    float sum = 0.f;
    for (auto &it : items) {
        it.second = expf((it.second - mx) * inv_t);
        sum += it.second;
    }
    size_t kept = items.size();
    if (top_p > 0.f && top_p < 1.f && kept > 1 && sum > 0.f) {
        float cum = 0.f;
        for (size_t i = 0; i < items.size(); ++i) {
            if (cum > top_p) {
                kept = i;
                break;
            }
            cum += items[i].second / sum;
        }
    }
    float ksum = 0.f;
    for (size_t i = 0; i < kept; ++i) ksum += items[i].second;
    std::uniform_real_distribution<float> U(0.f, 1.f);
    const float r = U(rng) * ksum;
    float acc = 0.f;
    for (size_t i = 0; i < kept; ++i) {
        acc += items[i].second;
        if (acc >= r) return items[i].first;
    }
    return items[0].first;
}

}  // namespace tb

struct tb_decoder : tb::Decoder {};

using namespace tb;

// RoPE tables as the reference builds them (src/llm/decoder.rs:334-350): f64
// freq = 1 / theta^(2i / hd), angle = pos * freq, cos/sin rounded to f32 and
// duplicated into both halves of each row.
static void rope_tables(std::vector<float> &c, std::vector<float> &s, int max_seq, int hd,
                        double theta) {
    const int half = hd / 2;
    c.assign((size_t)max_seq * hd, 0.f);
    s.assign((size_t)max_seq * hd, 0.f);
    for (int p = 0; p < max_seq; ++p)
        for (int i = 0; i < half; ++i) {
            const double freq = 1.0 / pow(theta, (2.0 * (double)i) / (double)hd);
            const double v = (double)p * freq;
            const float cv = (float)cos(v), sv = (float)sin(v);
            c[(size_t)p * hd + i] = c[(size_t)p * hd + i + half] = cv;
            s[(size_t)p * hd + i] = s[(size_t)p * hd + i + half] = sv;
        }
}

extern "C" {

int tb_decoder_create(const tb_decoder_config *cfg, const float *embed, const float *final_norm,
                      const void *lm_head_w, const float *lm_head_s, tb_decoder **out) {
    TB_REQUIRE(cfg && out && embed && final_norm && lm_head_w, TB_ERR_VALUE,
               "tb_decoder_create: null argument");
    *out = nullptr;
    const tb_decoder_config &c = *cfg;
    // Configuration checks of RustQwenDecoder::new (decoder.rs:214-233).
    TB_REQUIRE(c.hidden_size > 0 && c.hidden_size % 4 == 0, TB_ERR_VALUE,
               "hidden_size (" + std::to_string(c.hidden_size) + ") must be divisible by 4");
    TB_REQUIRE(c.group_size == 32 || c.group_size == 64 || c.weight_bits == 8, TB_ERR_VALUE,
               "group_size must be 32 or 64");
    TB_REQUIRE(c.weight_bits == 8 || c.hidden_size % c.group_size == 0, TB_ERR_VALUE,
               "hidden_size (" + std::to_string(c.hidden_size) +
                   ") must be divisible by group_size (" + std::to_string(c.group_size) + ")");
    TB_REQUIRE(c.head_dim > 0 && c.head_dim % 2 == 0, TB_ERR_VALUE,
               "head_dim (" + std::to_string(c.head_dim) + ") must be even");
    TB_REQUIRE(c.num_kv_heads > 0 && c.num_heads % c.num_kv_heads == 0, TB_ERR_VALUE,
               "num_heads (" + std::to_string(c.num_heads) +
                   ") must be divisible by num_kv_heads (" + std::to_string(c.num_kv_heads) + ")");
    TB_REQUIRE(c.weight_bits == 4 || c.weight_bits == 8, TB_ERR_VALUE, "weight_bits must be 4 or 8");
    TB_REQUIRE(c.lm_head_bits == 4 || c.lm_head_bits == 8 || c.lm_head_bits == 32, TB_ERR_VALUE,
               "lm_head_bits must be 4, 8 or 32");
    TB_REQUIRE(c.head_dim == 64 || c.head_dim == 128, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: head_dim must be 64 or 128");
    TB_REQUIRE(c.hidden_size % 32 == 0 && c.intermediate_size % 32 == 0 &&
                   (c.num_heads * c.head_dim) % 32 == 0,
               TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: hidden, intermediate and num_heads*head_dim must be multiples of 32");
    TB_REQUIRE(c.hidden_size <= kMaxHidden, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: hidden_size > " + std::to_string(kMaxHidden));
    TB_REQUIRE(c.max_seq_len > 0 && c.max_seq_len <= kMaxTiles * kAttnTile && c.vocab_size > 0 &&
                   c.num_layers > 0,
               TB_ERR_VALUE, "max_seq_len, vocab_size and num_layers must be positive");

    auto *d = new (std::nothrow) tb_decoder();
    TB_REQUIRE(d, TB_ERR_MEMORY, "Out of memory allocating the decoder");
    d->cfg = c;
    d->H = (int)c.hidden_size; d->I = (int)c.intermediate_size; d->hq = (int)c.num_heads;
    d->hkv = (int)c.num_kv_heads; d->hd = (int)c.head_dim; d->V = (int)c.vocab_size;
    d->L = (int)c.num_layers; d->max_seq = (int)c.max_seq_len; d->gs = (int)c.group_size;
    d->wbits = c.weight_bits; d->lmbits = c.lm_head_bits; d->eps = (float)c.rms_norm_eps;
    d->tq = (d->hq + 2 * d->hkv) * d->hd;
    d->v2 = d->wbits == 4 && d->gs == 64 && d->H % 64 == 0 && d->tq % 64 == 0 &&
            (d->hq * d->hd) % 64 == 0 && d->I % 64 == 0 && d->V % 64 == 0;
    d->nsplit = attn_nsplit(d->max_seq);
    d->hist_cap = d->max_seq;
    d->layers.resize(d->L);
    d->host_logits.assign(d->V, 0.f);
    int rc = TB_OK;
    auto bail = [&](int code) {
        delete d;
        return code;
    };
    if (hipGetDevice(&d->device) != hipSuccess) return bail(fail(TB_ERR_HIP, "no HIP device"));
    if (hipStreamCreateWithFlags(&d->st, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&d->ev0) != hipSuccess || hipEventCreate(&d->ev1) != hipSuccess)
        return bail(fail(TB_ERR_HIP, "stream/event creation failed"));
    if (hipHostMalloc((void **)&d->hstate, sizeof(DecState)) != hipSuccess)
        return bail(fail(TB_ERR_MEMORY, "pinned host allocation failed"));
    const size_t kv = (size_t)d->L * d->hkv * d->max_seq * d->hd * sizeof(float);
    if ((rc = d->upload(&d->embed, embed, (size_t)d->V * d->H * 4)) ||
        (rc = d->upload(&d->final_norm, final_norm, (size_t)d->H * 4)) ||
        (rc = d->alloc(&d->kc, kv)) || (rc = d->alloc(&d->vc, kv)) ||
        (rc = d->alloc(&d->x, d->H * 4)) || (rc = d->alloc(&d->xn, d->H * 4)) ||
        (rc = d->alloc(&d->qkv, d->tq * 4)) || (rc = d->alloc(&d->attn, d->hq * d->hd * 4)) ||
        (rc = d->alloc(&d->h, (size_t)d->I * 4)) || (rc = d->alloc(&d->logits, (size_t)d->V * 4)) ||
        (rc = d->alloc(&d->xa, (size_t)std::max({d->H, d->hq * d->hd, d->I}) * 4)) ||
        (rc = d->alloc(&d->part, (size_t)d->hq * d->nsplit * (d->hd + 4) * 4)) ||
        (rc = d->alloc(&d->am_v, kArgmaxBlocks * 4)) || (rc = d->alloc(&d->am_i, kArgmaxBlocks * 4)) ||
        (rc = d->alloc(&d->history, (size_t)d->hist_cap * 4)) ||
        (rc = d->alloc(&d->state, sizeof(DecState))) ||
        (rc = d->alloc(&d->xq_h, (size_t)(d->H / 32) * kXRecDwords * 4)) ||
        (rc = d->alloc(&d->xq_a, (size_t)(d->hq * d->hd / 32) * kXRecDwords * 4)) ||
        (rc = d->alloc(&d->xq_i, (size_t)(d->I / 32) * kXRecDwords * 4)) ||
        (rc = d->alloc(&d->ssq, (size_t)(d->H / 16) * 4)))
        return bail(rc);
    {
        const char *e = getenv("TB_DECODER_UNFUSED");
        d->fused = !(e && e[0] == '1');
        const char *j = getenv("TB_DECODER_J");
        if (j) sscanf(j, "%d,%d,%d,%d,%d", &d->rj[0], &d->rj[1], &d->rj[2], &d->rj[3], &d->rj[4]);
    }
    if (d->lmbits != 32)
        TB_REQUIRE(lm_head_s, TB_ERR_VALUE, "lm_head scales are required for a quantized lm_head");
    if (d->v2 && d->lmbits == 4) {
        if ((rc = d->upload_f16_scaled(&d->lm_w, &d->lm_s, lm_head_w, lm_head_s, d->V, d->H)))
            return bail(rc);
    } else {
        if ((rc = d->upload(&d->lm_w, lm_head_w, d->wbytes(d->lmbits, d->V, d->H)))) return bail(rc);
        if (d->lmbits != 32 &&
            (rc = d->upload(&d->lm_s, lm_head_s, d->sbytes(d->lmbits, d->V, d->H))))
            return bail(rc);
    }
    std::vector<float> ct, stb;
    rope_tables(ct, stb, d->max_seq, d->hd, c.rope_theta);
    if ((rc = d->upload(&d->cos_t, ct.data(), ct.size() * 4)) ||
        (rc = d->upload(&d->sin_t, stb.data(), stb.size() * 4)))
        return bail(rc);
    if (hipMemset(d->kc, 0, kv) != hipSuccess || hipMemset(d->vc, 0, kv) != hipSuccess ||
        hipMemset(d->x, 0, d->H * 4) != hipSuccess)
        return bail(fail(TB_ERR_HIP, "initial clear failed"));
    *out = d;
    return TB_OK;
}

int tb_decoder_set_layer(tb_decoder *d, int64_t layer, const float *in_norm, const void *qkv_w,
                         const float *qkv_s, const void *o_w, const float *o_s,
                         const float *post_norm, const void *gate_w, const float *gate_s,
                         const void *up_w, const float *up_s, const void *down_w,
                         const float *down_s, const float *qkv_b) {
    TB_REQUIRE(d, TB_ERR_VALUE, "null decoder");
    TB_REQUIRE(layer >= 0 && layer < d->L, TB_ERR_VALUE, "layer index out of range");
    TB_REQUIRE(in_norm && qkv_w && qkv_s && o_w && o_s && post_norm && gate_w && gate_s && up_w &&
                   up_s && down_w && down_s,
               TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: Each layer requires 12 tensors: input_norm, qkv_w, qkv_s, o_w, "
               "o_s, post_norm, gate_w, gate_s, up_w, up_s, down_w, down_s");
    Layer &y = d->layers[layer];
    TB_REQUIRE(!y.set, TB_ERR_VALUE, "decoder layer " + std::to_string(layer) + " set twice");
    const int b = d->wbits, H = d->H, I = d->I, qd = d->hq * d->hd;
    int rc;
    if ((rc = d->upload(&y.in_norm, in_norm, H * 4)) ||
        (rc = d->upload(&y.post_norm, post_norm, H * 4)) ||
        (rc = d->upload(&y.gate_w, gate_w, d->wbytes(b, I, H))) ||
        (rc = d->upload(&y.gate_s, gate_s, d->sbytes(b, I, H))) ||
        (rc = d->upload(&y.up_w, up_w, d->wbytes(b, I, H))) ||
        (rc = d->upload(&y.up_s, up_s, d->sbytes(b, I, H))))
        return rc;
    if (d->v2) {
        if ((rc = d->upload_f16_scaled(&y.qkv_w, &y.qkv_s, qkv_w, qkv_s, d->tq, H)) ||
            (rc = d->upload_f16_scaled(&y.o_w, &y.o_s, o_w, o_s, H, qd)) ||
            (rc = d->upload_f16_scaled(&y.down_w, &y.down_s, down_w, down_s, H, I)))
            return rc;
    } else if ((rc = d->upload(&y.qkv_w, qkv_w, d->wbytes(b, d->tq, H))) ||
               (rc = d->upload(&y.qkv_s, qkv_s, d->sbytes(b, d->tq, H))) ||
               (rc = d->upload(&y.o_w, o_w, d->wbytes(b, H, qd))) ||
               (rc = d->upload(&y.o_s, o_s, d->sbytes(b, H, qd))) ||
               (rc = d->upload(&y.down_w, down_w, d->wbytes(b, H, I))) ||
               (rc = d->upload(&y.down_s, down_s, d->sbytes(b, H, I)))) {
        return rc;
    }
    if (qkv_b && (rc = d->upload(&y.qkv_b, qkv_b, (size_t)d->tq * 4))) return rc;
    y.set = true;
    return TB_OK;
}

int tb_decoder_step(tb_decoder *d, int64_t token, int64_t offset, float *logits_out,
                    int64_t *argmax_out) {
    TB_REQUIRE(d, TB_ERR_VALUE, "null decoder");
    int rc = d->step(token, offset, logits_out != nullptr, argmax_out);
    if (rc) return rc;
    if (logits_out) memcpy(logits_out, d->host_logits.data(), (size_t)d->V * 4);
    return TB_OK;
}

int tb_decoder_decode_and_sample(tb_decoder *d, int64_t token, int64_t offset, float temperature,
                                 int64_t top_k, float repetition_penalty, const int64_t *recent,
                                 int64_t n_recent, float top_p, int64_t *token_out) {
    TB_REQUIRE(d && token_out, TB_ERR_VALUE, "null argument");
    const bool greedy = !std::isfinite(temperature) || temperature <= 0.f || top_k == 1;
    if (greedy && (repetition_penalty <= 1.0f || n_recent <= 0))
        return d->step(token, offset, false, token_out);
    if (d->device_samplable(temperature, top_k))
        return d->step_and_sample(token, offset, temperature, top_k, top_p, repetition_penalty,
                                  recent, n_recent, token_out);
    int rc = d->step(token, offset, true, nullptr);
    if (rc) return rc;
    tb::repetition_penalty(d->host_logits, recent, n_recent, repetition_penalty);
    *token_out = tb::sample(d->host_logits, temperature, top_k, top_p, d->rng);
    return TB_OK;
}

int tb_decoder_generate_sampled(tb_decoder *d, int64_t first_token, int64_t seq_len,
                                int64_t max_new_tokens, float temperature, int64_t top_k,
                                float repetition_penalty, float top_p, int64_t eos_token_id,
                                const int64_t *recent_seed, int64_t n_seed, int64_t *tokens_out,
                                int64_t *n_out, int64_t *seq_len_out) {
    TB_REQUIRE(d && tokens_out && n_out && seq_len_out, TB_ERR_VALUE, "null argument");
    TB_REQUIRE(seq_len >= 0 && max_new_tokens >= 0, TB_ERR_VALUE, "negative length");
    TB_REQUIRE(n_seed <= 0 || recent_seed, TB_ERR_VALUE, "null recent_seed");
    const bool greedy = !std::isfinite(temperature) || temperature <= 0.f || top_k == 1;
    if (greedy && repetition_penalty <= 1.0f)
        return tb_decoder_generate(d, first_token, seq_len, max_new_tokens, eos_token_id,
                                   tokens_out, n_out, seq_len_out);
    // generate_loop (decoder.rs:788-832) with its 64-token window (859-876):
    // push the token, decode it at seq_len + generated - 1, sample the next.
    std::vector<int64_t> win(recent_seed, recent_seed + std::max<int64_t>(n_seed, 0));
    auto push = [&](int64_t t) {
        win.push_back(t);
        if ((int64_t)win.size() > kSampleWindow) win.erase(win.begin(), win.end() - kSampleWindow);
    };
    int64_t n = 0, next = first_token;
    int rc;
    if (!d->device_samplable(temperature, top_k)) {
        while (n < max_new_tokens) {   // host sampler
            if (eos_token_id >= 0 && next == eos_token_id) break;
            tokens_out[n++] = next;
            push(next);
            if ((rc = d->step(next, seq_len + n - 1, true, nullptr))) return rc;
            tb::repetition_penalty(d->host_logits, win.data(), (int64_t)win.size(),
                                   repetition_penalty);
            next = tb::sample(d->host_logits, temperature, top_k, top_p, d->rng);
        }
    } else {
        // the parameters first: they pick the sampled graph's path
        if ((rc = d->set_sampler(temperature, top_k, top_p, repetition_penalty)) ||
            (rc = d->ensure_graph_s()))
            return rc;
        SampleWindow hw{};
        const int64_t w0 = std::min<int64_t>((int64_t)win.size(), kSampleWindow);
        hw.n = (int)w0;
        for (int64_t i = 0; i < w0; ++i) hw.tok[i] = win[win.size() - w0 + i];
        TB_HIP(hipMemcpyAsync(d->swin, &hw, sizeof(hw), hipMemcpyHostToDevice, d->st));
        // Steps inside the cache replay the sampling graph (window push,
        // penalty, draw and the next token all on the device); with an EOS
        // token each step's token is read back before the next.
        const int64_t valid = d->in_range(first_token, seq_len)
                                  ? std::min<int64_t>(max_new_tokens, d->max_seq - seq_len)
                                  : 0;
        if (valid > 0) {
            if ((rc = d->set_state((int)first_token, (int)seq_len))) return rc;
            if (eos_token_id < 0) {
                for (int64_t i = 0; i < valid; ++i) TB_HIP(hipGraphLaunch(d->sampled_graph(), d->st));
                std::vector<int> hist((size_t)valid);
                TB_HIP(hipMemcpyAsync(hist.data(), d->history, (size_t)valid * 4,
                                      hipMemcpyDeviceToHost, d->st));
                if ((rc = d->sampler_result(nullptr))) return rc;
                for (int64_t i = 0; i < valid; ++i) {
                    tokens_out[n++] = next;
                    next = hist[(size_t)i];
                }
            } else {
                while (n < valid && next != eos_token_id) {
                    tokens_out[n++] = next;
                    TB_HIP(hipGraphLaunch(d->sampled_graph(), d->st));
                    if ((rc = d->sampler_result(&next))) return rc;
                }
            }
            d->kv_used = std::max<int64_t>(d->kv_used, seq_len + n);
            // the device window now ends with the last decoded token
            const int64_t used = n;
            for (int64_t i = 0; i < used; ++i) push(tokens_out[i]);
        }
        // Positions past the cache: zeroed logits (decoder.rs:1066-1089), then
        // the penalty and the draw as for any step.
        while (n < max_new_tokens) {
            if (eos_token_id >= 0 && next == eos_token_id) break;
            tokens_out[n++] = next;
            push(next);
            if ((rc = d->step_and_sample(next, seq_len + n - 1, temperature, top_k, top_p,
                                         repetition_penalty, win.data(), (int64_t)win.size(),
                                         &next)))
                return rc;
        }
    }
    *n_out = n;
    *seq_len_out = seq_len + n;
    return TB_OK;
}

int tb_decoder_generate(tb_decoder *d, int64_t first_token, int64_t seq_len,
                        int64_t max_new_tokens, int64_t eos_token_id, int64_t *tokens_out,
                        int64_t *n_out, int64_t *seq_len_out) {
    TB_REQUIRE(d && tokens_out && n_out && seq_len_out, TB_ERR_VALUE, "null argument");
    TB_REQUIRE(seq_len >= 0 && max_new_tokens >= 0, TB_ERR_VALUE, "negative length");
    int rc = d->ensure_graph();
    if (rc) return rc;
    // Greedy generate_loop (decoder.rs:788-832): push the token, decode it at
    // seq_len + generated - 1, take the argmax as the next token.
    int64_t n = 0;
    const bool device_loop = eos_token_id < 0 && d->in_range(first_token, seq_len);
    if (device_loop) {
        // Steps whose position is inside the cache run as back-to-back graph
        // replays (token and position advance on the device); the reference
        // zeroes the logits of any later step, whose argmax is token 0.
        const int64_t valid = std::min<int64_t>(max_new_tokens, d->max_seq - seq_len);
        if (valid > 0) {
            rc = d->set_state((int)first_token, (int)seq_len);
            if (rc) return rc;
            for (int64_t i = 0; i < valid; ++i) TB_HIP(hipGraphLaunch(d->exec, d->st));
            std::vector<int> hist((size_t)valid);
            TB_HIP(hipMemcpyAsync(hist.data(), d->history, (size_t)valid * 4,
                                  hipMemcpyDeviceToHost, d->st));
            TB_HIP(hipStreamSynchronize(d->st));
            d->kv_used = std::max<int64_t>(d->kv_used, seq_len + valid);
            int64_t next = first_token;
            for (int64_t i = 0; i < max_new_tokens; ++i) {
                tokens_out[n++] = next;
                next = i < valid ? hist[(size_t)i] : 0;
            }
        } else {
            for (int64_t i = 0; i < max_new_tokens; ++i) tokens_out[n++] = i == 0 ? first_token : 0;
        }
    } else {
        int64_t next = first_token;
        while (n < max_new_tokens) {
            if (eos_token_id >= 0 && next == eos_token_id) break;
            tokens_out[n++] = next;
            int64_t am = 0;
            rc = d->step(next, seq_len + n - 1, false, &am);
            if (rc) return rc;
            next = am;
        }
    }
    *n_out = n;
    *seq_len_out = seq_len + n;
    return TB_OK;
}

// Leviathan acceptance of speculative_accept (decoder.rs:588-727) over the
// target rows [K, V] with the uniforms u[0..n_u) in order.
static int spec_accept(const float *rows, const int64_t *draft, const float *dprobs, int64_t K,
                       int64_t V, float temperature, float top_p, const double *u, int64_t n_u,
                       int64_t *accepted, int64_t *bonus) {
    int64_t ui = 0;
    auto next_u = [&]() { return ui < n_u ? u[ui++] : 0.0; };
    const float t = std::isfinite(temperature) && temperature > 0.f ? temperature : 1.0f;
    std::vector<float> tp((size_t)V);
    auto softmax = [&](const float *lg) {   // decoder.rs:624-641
        float m = -INFINITY;
        for (int64_t j = 0; j < V; ++j) m = std::max(m, std::isfinite(lg[j]) ? lg[j] : -INFINITY);
        float sum = 0.f;
        for (int64_t j = 0; j < V; ++j) {
            tp[j] = expf(((std::isfinite(lg[j]) ? lg[j] : -INFINITY) - m) / t);
            sum += tp[j];
        }
        const float inv = 1.0f / std::max(sum, 1e-30f);
        for (int64_t j = 0; j < V; ++j) tp[j] *= inv;
    };
    *accepted = 0;
    for (int64_t i = 0; i < K; ++i) {
        softmax(rows + (size_t)i * V);
        const int64_t d = std::min<int64_t>(std::max<int64_t>(draft[i], 0), V - 1);
        const float pt = tp[d], pd = std::max(dprobs[(size_t)i * V + d], 0.f);
        const float acc = std::min(pt / (pd + 1e-12f), 1.0f);
        if (next_u() <= (double)acc) {
            *accepted += 1;
            continue;
        }
        // rejected: resample from max(0, p_target - p_draft) (decoder.rs:677-702)
        std::vector<float> c((size_t)V);
        float sc = 0.f;
        for (int64_t j = 0; j < V; ++j) {
            c[j] = std::max(tp[j] - dprobs[(size_t)i * V + j], 0.f);
            sc += c[j];
        }
        if (sc > 1e-12f) {
            const float r = (float)next_u() * sc;
            float a = 0.f;
            *bonus = V - 1;
            for (int64_t j = 0; j < V; ++j) {
                a += c[j];
                if (a >= r) {
                    *bonus = j;
                    break;
                }
            }
        } else {
            int64_t bj = 0;
            for (int64_t j = 1; j < V; ++j)
                if (tp[j] > tp[bj]) bj = j;
            *bonus = bj;
        }
        return TB_OK;
    }
    // all accepted: the bonus from the last row with the nucleus
    // (decoder.rs:705-726), candidates by probability (ties: lower index)
    softmax(rows + (size_t)(K - 1) * V);
    std::vector<int64_t> idx((size_t)V);
    for (int64_t j = 0; j < V; ++j) idx[j] = j;
    std::stable_sort(idx.begin(), idx.end(), [&](int64_t a, int64_t b) { return tp[a] > tp[b]; });
    int64_t kept = V;
    if (top_p > 0.f && top_p < 1.f) {
        float cum = 0.f;
        for (int64_t i = 0; i < V; ++i) {
            if (cum > top_p) {
                kept = i;
                break;
            }
            cum += tp[idx[i]];
        }
        kept = std::max<int64_t>(kept, 1);
    }
    float mass = 0.f;
    for (int64_t i = 0; i < kept; ++i) mass += tp[idx[i]];
    const float r = (float)next_u() * std::max(mass, 1e-30f);
    float a = 0.f;
    *bonus = idx[kept - 1];
    for (int64_t i = 0; i < kept; ++i) {
        a += tp[idx[i]];
        if (a >= r) {
            *bonus = idx[i];
            break;
        }
    }
    return TB_OK;
}

// The decoder's f64 uniforms for speculative acceptance: 53 bits of the same
// splitmix64 stream as the sampler's draws.
static double spec_uniform(uint64_t seed, uint64_t counter) {
    uint64_t x = seed + (counter + 1ull) * 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    x ^= x >> 31;
    return (double)(x >> 11) / 9007199254740992.0;
}

double tb_spec_uniform(uint64_t seed, uint64_t counter) { return spec_uniform(seed, counter); }

int tb_speculative_accept_rows(const float *target_rows, const int64_t *draft_tokens,
                               const float *draft_probs, int64_t k, int64_t vocab,
                               float temperature, float top_p, const double *u, int64_t n_u,
                               int64_t *accepted, int64_t *bonus) {
    TB_REQUIRE(accepted && bonus, TB_ERR_VALUE, "null argument");
    TB_REQUIRE(vocab > 0 && k >= 0, TB_ERR_VALUE, "bad shape");
    if (k == 0) {
        *accepted = 0;
        *bonus = vocab - 1;
        return TB_OK;
    }
    TB_REQUIRE(target_rows && draft_tokens && draft_probs && (n_u == 0 || u), TB_ERR_VALUE,
               "null argument");
    return spec_accept(target_rows, draft_tokens, draft_probs, k, vocab, temperature, top_p, u,
                       n_u, accepted, bonus);
}

int tb_decoder_verify(tb_decoder *d, int64_t start_offset, const int64_t *tokens, int64_t n,
                      float *logits_out) {
    TB_REQUIRE(d && (n == 0 || (tokens && logits_out)), TB_ERR_VALUE, "null argument");
    TB_REQUIRE(start_offset >= 0 && start_offset + n <= d->max_seq, TB_ERR_VALUE,
               "verify exceeds max_seq_len");
    if (n == 0) return TB_OK;
    bool batch = d->wbits == 4 && n >= 2 && d->under_cap(start_offset, n) && !d->a8_wanted();
    for (int64_t i = 0; i < n && batch; ++i) batch = tokens[i] >= 0 && tokens[i] < d->V;
    if (!batch) {
        for (int64_t i = 0; i < n; ++i) {
            int rc = d->step(tokens[i], start_offset + i, true, nullptr);
            if (rc) return rc;
            memcpy(logits_out + (size_t)i * d->V, d->host_logits.data(), (size_t)d->V * 4);
        }
        return TB_OK;
    }
    // verify_tokens (decoder.rs:565-581) as one batched forward over the n
    // positions: the weights are read once, not n times.
    int rc;
    if (n > d->pf_rows_n) {
        if ((rc = d->alloc(&d->pf_rows, (size_t)n * d->V * 4))) return rc;
        d->pf_rows_n = n;
    }
    if ((rc = d->prefill_batched(tokens, n, start_offset, d->pf_rows))) return rc;
    TB_HIP(hipMemcpy(logits_out, d->pf_rows, (size_t)n * d->V * 4, hipMemcpyDeviceToHost));
    return TB_OK;
}

int tb_decoder_speculative_accept(tb_decoder *d, int64_t offset, const int64_t *draft_tokens,
                                  int64_t k, const float *draft_probs, float temperature,
                                  float top_p, int64_t *accepted, int64_t *bonus) {
    TB_REQUIRE(d && accepted && bonus, TB_ERR_VALUE, "null argument");
    if (k == 0) {
        *accepted = 0;
        *bonus = d->V - 1;
        return TB_OK;
    }
    TB_REQUIRE(draft_tokens && draft_probs, TB_ERR_VALUE, "draft_probs must be K×V row-major");
    // step_internal zeroes the logits of positions past the cache and changes
    // nothing else (decoder.rs:1066-1089), so the reference's acceptance runs on
    // zero rows there instead of failing: verify only the positions inside.
    std::vector<float> rows((size_t)k * d->V, 0.f);
    const int64_t inside = std::max<int64_t>(0, std::min<int64_t>(k, d->max_seq - offset));
    if (inside > 0) {
        int rc = tb_decoder_verify(d, offset, draft_tokens, inside, rows.data());
        if (rc) return rc;
    }
    std::vector<double> u((size_t)k + 1);
    for (auto &v : u) v = spec_uniform(d->seed, d->draws++);
    return spec_accept(rows.data(), draft_tokens, draft_probs, k, d->V, temperature, top_p,
                       u.data(), (int64_t)u.size(), accepted, bonus);
}

int tb_decoder_prefill(tb_decoder *d, const int64_t *tokens, int64_t n, int64_t start_offset,
                       int64_t *offset_out) {
    TB_REQUIRE(d && offset_out, TB_ERR_VALUE, "null argument");
    if (n <= 0) {
        *offset_out = start_offset;
        return TB_OK;
    }
    TB_REQUIRE(tokens, TB_ERR_VALUE, "null tokens");
    TB_REQUIRE(start_offset >= 0 && start_offset + n <= d->max_seq, TB_ERR_VALUE,
               "prefill " + std::to_string(n) + " tokens at offset " + std::to_string(start_offset) +
                   " exceeds max_seq_len " + std::to_string(d->max_seq));
    if (d->prefill_batchable(tokens, n, start_offset)) {
        int rc = d->prefill_batched(tokens, n, start_offset);
        if (rc) return rc;
    } else {
        for (int64_t i = 0; i < n; ++i) {
            int rc = d->step(tokens[i], start_offset + i, i + 1 == n, nullptr);
            if (rc) return rc;
        }
    }
    *offset_out = start_offset + n;
    return TB_OK;
}

int tb_decoder_reset_kv(tb_decoder *d) {
    TB_REQUIRE(d, TB_ERR_VALUE, "null decoder");
    const size_t kv = (size_t)d->L * d->hkv * d->max_seq * d->hd * sizeof(float);
    if (d->kv_used > 0) {
        TB_HIP(hipMemsetAsync(d->kc, 0, kv, d->st));
        TB_HIP(hipMemsetAsync(d->vc, 0, kv, d->st));
        TB_HIP(hipStreamSynchronize(d->st));
    }
    d->kv_used = 0;
    return TB_OK;
}

int tb_decoder_copy_kv(tb_decoder *d, int64_t layer, const float *k, const float *v,
                       int64_t src_max, int64_t seq_len) {
    TB_REQUIRE(d && k && v, TB_ERR_VALUE, "null argument");
    TB_REQUIRE(layer >= 0 && layer < d->L, TB_ERR_VALUE, "layer index out of range");
    TB_REQUIRE(seq_len >= 0 && seq_len <= src_max && seq_len <= d->max_seq, TB_ERR_VALUE,
               "KV cache copy out of bounds");
    // Source [hkv, src_max, hd] per layer (decoder.rs:479-523).
    const size_t row = (size_t)d->hd * 4;
    for (int hh = 0; hh < d->hkv; ++hh) {
        const size_t so = (size_t)hh * src_max * d->hd;
        const size_t dof = ((size_t)layer * d->hkv + hh) * d->max_seq * d->hd;
        TB_HIP(hipMemcpyAsync(d->kc + dof, k + so, row * seq_len, hipMemcpyDefault, d->st));
        TB_HIP(hipMemcpyAsync(d->vc + dof, v + so, row * seq_len, hipMemcpyDefault, d->st));
    }
    TB_HIP(hipStreamSynchronize(d->st));
    d->kv_used = std::max<int64_t>(d->kv_used, seq_len);
    return TB_OK;
}

int tb_decoder_kv_len(tb_decoder *d, int64_t *out) {
    TB_REQUIRE(d && out, TB_ERR_VALUE, "null argument");
    *out = d->kv_used;
    return TB_OK;
}

int tb_decoder_get_logits(tb_decoder *d, float *out) {
    TB_REQUIRE(d && out, TB_ERR_VALUE, "null argument");
    memcpy(out, d->host_logits.data(), (size_t)d->V * 4);
    return TB_OK;
}

int tb_decoder_set_seed(tb_decoder *d, uint64_t seed) {
    TB_REQUIRE(d, TB_ERR_VALUE, "null decoder");
    d->rng.seed(seed);
    d->seed = seed;
    d->draws = 0;
    return TB_OK;
}

int tb_decoder_set_attention_cap(tb_decoder *d, int64_t cap) {
    TB_REQUIRE(d, TB_ERR_VALUE, "null decoder");
    TB_REQUIRE(cap >= 0, TB_ERR_VALUE, "attention cap must be >= 0 (0: none)");
    const int c = (cap == 0 || cap > INT_MAX) ? INT_MAX : (int)cap;
    if (c == d->attn_cap) return TB_OK;
    TB_HIP(hipStreamSynchronize(d->st));
    d->attn_cap = c;
    return d->drop_graphs();   // the captured steps hold the old cap
}

int tb_decoder_set_rope_tables(tb_decoder *d, const float *cos_t, const float *sin_t,
                               int64_t rows, int64_t head_dim) {
    TB_REQUIRE(d, TB_ERR_VALUE, "null decoder");
    TB_REQUIRE(cos_t && sin_t, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: set_rope_tables: null table");
    TB_REQUIRE(rows == d->max_seq && head_dim == d->hd, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: set_rope_tables: tables must be [max_seq_len=" +
                   std::to_string(d->max_seq) + ", head_dim=" + std::to_string(d->hd) + "]");
    const size_t bytes = (size_t)rows * (size_t)head_dim * sizeof(float);
    // The step graphs read the tables through these same buffers.
    TB_HIP(hipStreamSynchronize(d->st));
    TB_HIP(hipMemcpy(d->cos_t, cos_t, bytes, hipMemcpyDefault));
    TB_HIP(hipMemcpy(d->sin_t, sin_t, bytes, hipMemcpyDefault));
    return TB_OK;
}

int tb_decoder_time_greedy(tb_decoder *d, int64_t first_token, int64_t offset, int64_t n_steps,
                           float *ms_out) {
    TB_REQUIRE(d && ms_out, TB_ERR_VALUE, "null argument");
    TB_REQUIRE(d->in_range(first_token, offset) && offset + n_steps <= d->max_seq, TB_ERR_VALUE,
               "timed steps must stay inside the KV cache");
    int rc = d->ensure_graph();
    if (rc) return rc;
    rc = d->set_state((int)first_token, (int)offset);
    if (rc) return rc;
    TB_HIP(hipEventRecord(d->ev0, d->st));
    for (int64_t i = 0; i < n_steps; ++i) TB_HIP(hipGraphLaunch(d->exec, d->st));
    TB_HIP(hipEventRecord(d->ev1, d->st));
    TB_HIP(hipEventSynchronize(d->ev1));
    TB_HIP(hipEventElapsedTime(ms_out, d->ev0, d->ev1));
    d->kv_used = std::max<int64_t>(d->kv_used, offset + n_steps);
    return TB_OK;
}

int tb_decoder_destroy(tb_decoder *d) {
    delete d;
    return TB_OK;
}

}  // extern "C"

// Launchers of the decoder-step kernels (decode.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tb {

// Device-resident step state: every step kernel reads token / pos from here,
// and the greedy argmax writes the next token and advances pos and step.
struct DecState {
    int token;    // input token of the step
    int pos;      // its position (offset); the step attends over 0..pos
    int step;     // index into the greedy history
    int argmax;   // argmax of the last step's logits
};

constexpr int kMaxHidden = 8192;   // largest hidden size the decoder accepts
constexpr int kNormChunks = 32;    // 32-element chunks normalised per RMSNorm block
constexpr int kAttnTile = 64;      // KV positions per attention block
constexpr int kArgmaxBlocks = 256;
constexpr int kMaxTiles = 1024;     // max_seq_len <= kMaxTiles * kAttnTile
// Attention blocks per KV head: a longer cache has each block fold several
// tiles, so the grid and the merge stay this size whatever max_seq_len is.
constexpr int kAttnMaxSplits = 128;

int launch_rmsnorm(const DecState *st, const float *embed, float *x, const float *w, float *xn,
                   uint32_t *xq, int H, float eps, hipStream_t s);
// x = embed[token]; x * w in f32 (xw) and as records (xq); 16-element sums of
// squares of x (the fused-RMSNorm step's first input).
int launch_embed_rec(const DecState *st, const float *embed, float *x, const float *w,
                     float *xw, uint32_t *xq, float *ssq, int H, hipStream_t s);
int launch_rope_kv(const DecState *st, float *qkv, const float *cos_t, const float *sin_t,
                   float *kc, float *vc, int hq, int hkv, int hd, int max_seq, hipStream_t s);
int attn_nsplit(int max_seq);
// part: [hq][attn_nsplit(max_seq)][hd + 4] floats of scratch.  The step at
// position pos attends positions 0 .. min(pos + 1, cap) - 1: the native step
// scores at most the first kNativeAttnCap positions (decoder.rs:1179-1184),
// the per-layer path every position (cap = INT_MAX).
constexpr int kNativeAttnCap = 32768;
int launch_attention(const DecState *st, const float *qkv, const float *kc, const float *vc,
                     float *part, float *out, uint32_t *xq, int hq, int hkv, int hd, int max_seq,
                     int cap, hipStream_t s);
// Batched prefill: M consecutive positions start .. start+M-1.
int launch_embed_rows(const int *tok, const float *embed, float *X, int M, int H, hipStream_t s);
int launch_rmsnorm_rows(const float *X, const float *w, float *Xn, int M, int H, float eps,
                        hipStream_t s);
// qkv [M][(hq + 2 hkv) hd] -> q [M][hq][hd] rotated; k (rotated) and v into the caches.
int launch_rope_rows(const float *qkv, float *q, float *kc, float *vc, const float *cos_t,
                     const float *sin_t, int start, int M, int hq, int hkv, int hd, int max_seq,
                     hipStream_t s);
// Causal attention of the M rows of q over cache positions 0 .. start + m; out [M][hq hd].
// With scratch (prefill_attention_scratch bytes) the key range is split over
// blocks when few query tiles meet a long cache; without, one block per tile
// and KV head walks the whole range.
int prefill_attention_splits(int start, int M, int hq, int hkv);
size_t prefill_attention_scratch(int M, int hq, int hd, int nsplit);
int launch_prefill_attention(const float *q, const float *kc, const float *vc, float *out,
                             int start, int M, int hq, int hkv, int hd, int max_seq,
                             float *scratch, hipStream_t s);
int launch_argmax(const float *logits, int n, float *pv, int *pi, DecState *st, int *history,
                  int hist_cap, hipStream_t s);

}  // namespace tb

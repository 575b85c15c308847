/*
 * tbhip.h -- C ABI of libtbhip.so, the gfx950 (MI355X) implementation of
 * TorchBurn's quantized decode hot path.
 *
 * Every entry point returns a status code (TB_OK == 0) and never throws.  On
 * failure tb_last_error() returns the message of the last failing call on the
 * calling thread.  The status codes keep the reference's error split:
 *   TB_ERR_UNSUPPORTED  <- UnsupportedOpError, "TB_UNSUPPORTED:" marker
 *                          (reference src/dlpack.rs:35-53; shape checks such as
 *                          src/quantization/packed_v2.rs:577-596)
 *   TB_ERR_VALUE        <- ValueError (src/llm/decoder.rs:214-233, 435-442)
 *   TB_ERR_MEMORY       <- MemoryError (src/llm/decoder.rs:238-246)
 *   TB_ERR_HIP          <- a HIP runtime failure (no reference counterpart)
 *
 * Pointer convention.  Stateless ops take DEVICE pointers (HBM-resident
 * tensors, row-major, contiguous) and a hipStream_t passed as void* (NULL = the
 * default stream); they are asynchronous on that stream.
 *
 * Scratch.  An op that needs scratch (activation records, h, split-K
 * partials) takes it from a workspace owned by the library per (device,
 * stream): calls on different streams or threads never share scratch, and
 * calls on one stream are ordered by that stream.  A workspace only grows; a
 * buffer it outgrows is kept, not freed, until the process ends, so a graph
 * captured earlier still points at valid memory.  Growth may happen while the
 * stream is being captured (this thread's capture mode is relaxed around the
 * allocation).  tb_fused_swiglu_mlp_w4a32_noalloc uses a fixed static scratch
 * instead and allocates nothing.
 *
 * The decoder copies HOST weights to the device once at creation, as
 * RustQwenDecoder::new copies them into Rust-owned memory
 * (src/llm/decoder.rs:235-332).  A decoder handle is not thread-safe, matching
 * the reference's &mut self receivers.
 *
 * Weight layouts are the reference's:
 *   INT4 grouped ("v1", python/torchburn/quantization.py:53-118):
 *     w u8 [N, ceil(K/2)]: byte j of a row holds element 2j in its low nibble
 *     and 2j+1 in its high nibble, each stored as q + 8, q in [-8, 7];
 *     scales f32 [N, ceil(K/group_size)].
 *   INT8 per-channel (src/quantization/fused_ops.rs:554-589):
 *     w i8 [N, K]; scales f32 [N] (or [1] for one per-tensor scale).
 */
#ifndef TBHIP_H
#define TBHIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define TB_API __attribute__((visibility("default")))
#else
#define TB_API
#endif

#define TB_OK 0
#define TB_ERR_UNSUPPORTED 1
#define TB_ERR_VALUE 2
#define TB_ERR_MEMORY 3
#define TB_ERR_HIP 4

/* Message of the last failing call on this thread ("" if none). */
TB_API const char *tb_last_error(void);

/* Library version string and the device architecture it was built for. */
TB_API const char *tb_version(void);

/*
 * out[m, n] = sum_g s[n, g] * sum_{i in g} (nib(w[n, i]) - 8) * x[m, i] + bias[n]
 *
 * Replaces the reference's w4a32_grouped_linear: the PyO3 binding
 * src/ffi/quantization_ffi.rs:56-85 -> src/quantization/packed_v2.rs:557-624
 * -> gemm_w4a32_grouped / gemv_w4a32_grouped (src/quantization/gemv.rs:1514-1725).
 * x f32 [M, K], w u8 [N, ceil(K/2)], scales f32 [N, ceil(K/gs)], bias f32 [N]
 * or NULL, out f32 [M, N].  Any K >= 1 and any even group_size (a short last
 * group, as gemv.rs:1650-1660; groups start on byte boundaries).  K a multiple of 32 with a power-of-two group_size >= 32
 * dividing K runs the streaming kernels: M <= 4 the GEMV (one pass of up to 4
 * rows, K <= 16384), M >= 5 the FP32-MFMA projection (weights dequantized in
 * registers into the MFMA operand); other shapes run the any-shape GEMV.
 */
TB_API int tb_w4a32_grouped_linear(const float *x, const uint8_t *w_packed, const float *scales,
                            const float *bias, float *out, int64_t m, int64_t n, int64_t k,
                            int64_t group_size, void *stream);

/*
 * The v2 layout (src/quantization/packed_v2.rs:26-143): each 64-element group
 * of a row is one 34-byte block, 32 bytes of v1 nibbles then the group scale as
 * little-endian IEEE binary16.
 *
 * out[m, n] = sum_g f16(block[n, g]) * sum_{i in g} (nib - 8) * x[m, i] + bias[n]:
 * the reference's w4a32_grouped_linear_v2 (binding
 * src/ffi/quantization_ffi.rs:87-108 -> src/quantization/packed_v2.rs:489-553
 * -> gemv_w4a32_grouped_v2, packed_v2.rs:326-485).  w_blocked u8 [N, (K/64)*34]
 * (4-byte aligned); group_size must be 64 and K a multiple of 64 (the
 * reference's quantizer requires both, python/torchburn/quantization.py:121-152).
 */
TB_API int tb_w4a32_grouped_linear_v2(const float *x, const uint8_t *w_blocked, const float *bias,
                                      float *out, int64_t m, int64_t n, int64_t k,
                                      int64_t group_size, void *stream);

/*
 * v1 nibbles [N, K/2] + f32 scales [N, K/64] -> v2 blocks [N, (K/64)*34], the
 * scales rounded to binary16 to nearest even: pack_rows_w4a32_group64_v1_to_v2
 * (src/quantization/packed_v2.rs:114-143, f32_to_f16 66-105), run on the device.
 */
TB_API int tb_pack_rows_w4a32_group64_v1_to_v2(const uint8_t *w_packed, const float *scales,
                                               uint8_t *out, int64_t n, int64_t k, void *stream);

/*
 * v2 blocks [N, (K/64)*34] -> f32 weights [N, K], (nib - 8) * f16 scale:
 * dequantize_int4_grouped_v2 (python/torchburn/quantization.py:155-169).
 */
TB_API int tb_dequantize_int4_grouped_v2(const uint8_t *w_blocked, float *out, int64_t n,
                                         int64_t k, void *stream);

/*
 * f32 weights [N, K] -> v1 nibbles [N, K/2] + f32 scales [N, K/gs] on the device:
 * quantize_weight_int4_grouped (python/torchburn/quantization.py:53-118),
 * s = max(max|w| / 7, 1e-8) per group, q = clamp(round_half_even(w / s), -8, 7).
 * Any group_size >= 1 that divides K (TB_ERR_VALUE with the reference's
 * message otherwise); an odd K is TB_ERR_VALUE (the reference's nibble pairs
 * do not line up there and torch raises).
 */
TB_API int tb_quantize_weight_int4_grouped(const float *w, uint8_t *packed, float *scales,
                                           int64_t n, int64_t k, int64_t group_size,
                                           void *stream);

/*
 * f32 weights [N, K] -> int8 [N, K] + per-row f32 scales [N] on the device:
 * quantize_linear_weights_int8 (binding src/ffi/quantization_ffi.rs:258-269 ->
 * src/quantization/fused_ops.rs:554-589), s = max|w| / 127 (1 when max|w| <= 1e-8),
 * q = clamp(round_half_away(w * (1 / s)), -127, 127).
 */
TB_API int tb_quantize_weight_int8(const float *w, int8_t *q, float *scales, int64_t n,
                                   int64_t k, void *stream);

/*
 * v2 blocks [N, (K/64)*34] -> v1 nibbles [N, K/2] + f32 scales [N, K/64]: the
 * quantized-cache migration of the reference's loader
 * (python/torchburn/llm/loader.py:540-561), on the device.
 */
TB_API int tb_unpack_rows_w4a32_group64_v2_to_v1(const uint8_t *w_blocked, uint8_t *w_packed,
                                                 float *scales, int64_t n, int64_t k,
                                                 void *stream);

/*
 * Token sampling on the device over device logits [vocab]: apply_repetition_penalty
 * (src/llm/decoder.rs:878-899; logits modified in place, recent: device int64
 * [n_recent], each distinct in-vocabulary token once) then sample_logits
 * (decoder.rs:908-1020): greedy when temperature is not finite or <= 0 or
 * top_k == 1, else the top-k (ties: lower index first; non-finite logits as
 * -inf), softmax at the temperature, nucleus cut at top_p, one draw.  The
 * reference draws from an unseeded generator; here draw number `counter` of
 * `seed` is u = tb_sample_uniform(seed, counter).  Any top_k (above 128 one
 * block takes the whole vocabulary and finds the cut and the draw by radix
 * searches over the sorted mass); vocab <= 262144.  Synchronizes the stream;
 * *token_out and *u_out (or -1 when nothing was drawn) are host values.
 */
TB_API int tb_sample_logits(float *logits, int64_t vocab, float temperature, int64_t top_k,
                            float top_p, float repetition_penalty, const int64_t *recent,
                            int64_t n_recent, uint64_t seed, uint64_t counter, int64_t *token_out,
                            float *u_out, void *stream);

/* The uniform in [0, 1) (24 bits) of draw `counter` under `seed`: splitmix64. */
TB_API float tb_sample_uniform(uint64_t seed, uint64_t counter);

/*
 * Selects the reference's AVX-512 VNNI-tier semantics for group-64 INT4
 * projections: each activation row is quantized to bytes, s_x = max(max|x|,
 * 1e-10) / 127, q = round-half-even(x * (1 / s_x)) for the first 16 * (K / 16)
 * elements and round-half-away(x / s_x) for the rest
 * (src/quantization/gemv.rs:1353-1389), and contracted with the nibbles
 * (gemv.rs:1422-1473, packed_v2.rs:204-323).  It reaches every group-64 INT4
 * projection the reference runs through those kernels: the linear entries
 * (tb_w4a32_grouped_linear[_residual], _v2), the fused SwiGLU MLP (x before
 * the gate / up pair, h before down: fused_ops.rs:215-232, 409-421), the
 * per-layer steps (fused_ops.rs:932-1049, fused_transformer.rs:102-299) and the
 * decoder (QKV, O, gate / up, down and an INT4 lm_head: decoder.rs:1029-1049,
 * 1262-1282; a decoder re-captures its step when the setting changes, and
 * prefills and verifies step by step while it is on).  The reference picks
 * this by CPU feature (gemv.rs:1541-1563); 0 (the default) is its exact W4A32
 * result.  Returns the previous setting.  Process-wide.
 */
TB_API int tb_set_vnni_semantics(int enabled);

/* Frees the workspace the library keeps for `stream` on the current device (and
 * the smaller buffers it replaced), for callers that create streams per request
 * and would otherwise hold one workspace per stream until the process ends.  No
 * reference counterpart (the reference allocates per call).  It waits for the
 * device to finish its work first; a graph captured on that stream that used the
 * library must not be replayed afterwards.  A later call on the stream gets a
 * new workspace.  TB_OK when the stream has none. */
TB_API int tb_release_stream_workspace(void *stream);

/*
 * out = residual + w4a32_grouped_linear(x, ...).  The reference performs the
 * residual add as a separate pass after the projection
 * (src/llm/decoder.rs:1235-1238 and 1344-1347, fast_vector_add at
 * src/quantization/fused_ops.rs:1121-1185); here it is the GEMV's epilogue.
 * residual and out are f32 [M, N]; out may alias residual.
 */
TB_API int tb_w4a32_grouped_linear_residual(const float *x, const uint8_t *w_packed,
                                     const float *scales, const float *bias,
                                     const float *residual, float *out, int64_t m, int64_t n,
                                     int64_t k, int64_t group_size, void *stream);

/*
 * h[m, j] = silu(gate_j . x_m + gate_b[j]) * (up_j . x_m + up_b[j]), with
 * silu(g) = g / (1 + exp(-g)): the neuron loop of fused_swiglu_mlp_w4a32
 * (src/quantization/fused_ops.rs:244-407; neuron kernels
 * src/quantization/gemv/swiglu.rs:205-289).  gate_b / up_b may be NULL.
 * x f32 [M, K]; gate_w/up_w u8 [I, K/2]; gate_s/up_s f32 [I, K/gs]; h f32 [M, I].
 */
TB_API int tb_swiglu_w4a32(const float *x, const uint8_t *gate_w, const float *gate_s,
                    const float *gate_b, const uint8_t *up_w, const float *up_s,
                    const float *up_b, float *h, int64_t m, int64_t k, int64_t inter,
                    int64_t group_size, void *stream);

/*
 * out = [residual +] down(silu(gate(x)) * up(x)): the reference's
 * fused_swiglu_mlp_w4a32 (binding src/ffi/quantization_ffi.rs:203-256,
 * kernel src/quantization/fused_ops.rs:138-424), with the residual add of
 * src/llm/decoder.rs:1344-1347 folded in when residual != NULL.
 * The intermediate h [M, I] lives in a device workspace owned by the library
 * (allocated on first use, grown on demand, freed at process exit).
 */
TB_API int tb_fused_swiglu_mlp_w4a32(const float *x, const uint8_t *gate_w, const float *gate_s,
                              const float *gate_b, const uint8_t *up_w, const float *up_s,
                              const float *up_b, const uint8_t *down_w, const float *down_s,
                              const float *down_b, const float *residual, float *out,
                              int64_t m, int64_t k, int64_t inter, int64_t n_out,
                              int64_t group_size, void *stream);

/*
 * tb_fused_swiglu_mlp_w4a32 without any allocation, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * intermediates (h, the x / h records, the split-K partials) live in a 16 MiB
 * static device array, one per GPU, instead of the per-stream workspace:
 * shapes needing more return TB_ERR_UNSUPPORTED with the byte count before any
 * GPU work (the Llama-3-8B MLP fits at M = 1..54 and 65..88; M = 55..64 and
 * M >= 89 are refused: the split-K partials and the records of the batched
 * projection grow with the row tiles).  Every call on one GPU shares that array, so calls that overlap on
 * one GPU (two streams, or two threads) race; nothing in it needs clearing
 * between calls.  Same arguments and results as tb_fused_swiglu_mlp_w4a32.
 */
TB_API int tb_fused_swiglu_mlp_w4a32_noalloc(const float *x, const uint8_t *gate_w,
                                             const float *gate_s, const float *gate_b,
                                             const uint8_t *up_w, const float *up_s,
                                             const float *up_b, const uint8_t *down_w,
                                             const float *down_s, const float *down_b,
                                             const float *residual, float *out, int64_t m,
                                             int64_t k, int64_t inter, int64_t n_out,
                                             int64_t group_size, void *stream);

/*
 * Activation chunk records, for callers that reuse one x across several INT4
 * projections (no reference counterpart: the reference converts x inside each
 * GEMV).  A record holds 32 activations as 24-bit fixed-point integers in six
 * 4-bit limb planes plus a power-of-two step and an integer sum per 16-element
 * half: 112 bytes per 32 elements, tb_x_records_bytes(m, k) in total, laid out per row as 7 planes
 * of 16 bytes per chunk.  The layout is internal to this library.  tb_xquant builds them from x [M, K];
 * the *_xq GEMVs read them instead of building their own (x itself is still
 * read when a chunk holds NaN/Inf).  residual may be NULL.
 */
TB_API int64_t tb_x_records_bytes(int64_t m, int64_t k);
TB_API int tb_xquant(const float *x, uint32_t *xq, int64_t m, int64_t k, void *stream);
TB_API int tb_w4a32_gemv_xq(const float *x, const uint32_t *xq, const uint8_t *w_packed,
                            const float *scales, const float *bias, const float *residual,
                            float *out, int64_t m, int64_t n, int64_t k, int64_t group_size,
                            void *stream);
TB_API int tb_swiglu_w4a32_xq(const float *x, const uint32_t *xq, const uint8_t *gate_w,
                              const float *gate_s, const float *gate_b, const uint8_t *up_w,
                              const float *up_s, const float *up_b, float *h, int64_t m,
                              int64_t k, int64_t inter, int64_t group_size, void *stream);

/*
 * out[m, n] = (sum_k (nib(w[n, k]) - 8) * x[m, k]) * s[n] + bias[n]: the
 * reference's per-channel w4a32_linear (binding src/ffi/quantization_ffi.rs:32-54,
 * kernel src/quantization/gemv.rs:1066-1182; dispatched by the compile engine,
 * src/engine/dispatch_op/d_quant.rs:109-125).  w u8 [N, ceil(K/2)] (v1 nibbles),
 * s_len 1 (one per-tensor scale) or N; bias NULL or [N]; any K.
 */
TB_API int tb_w4a32_linear(const float *x, const uint8_t *w_packed, const float *scales,
                           int64_t s_len, const float *bias, float *out, int64_t m, int64_t n,
                           int64_t k, void *stream);

/*
 * f32 weights [N, K] -> v1 nibbles [N, ceil(K/2)] + one f32 scale per row [N] on
 * the device: quantize_linear_weights_int4 (binding quantize_linear_int4,
 * python/torchburn/quantization.py:44-50 -> src/quantization/fused_ops.rs:592-639),
 * s = max|w| / 7 (1 when max|w| <= 1e-8), q = clamp(round_half_away(w * (1 / s)),
 * -8, 7); an odd K pads the last byte with the nibble 8.
 */
TB_API int tb_quantize_weight_int4(const float *w, uint8_t *packed, float *scales, int64_t n,
                                   int64_t k, void *stream);

/*
 * out[m, n] = (sum_k x[m, k] * w[n, k]) * s[n] + bias[n]: the reference's
 * w8a32_linear (binding src/ffi/quantization_ffi.rs:8-30, kernel
 * src/quantization/gemv.rs:733-1061).  w i8 [N, K]; s_len 1 (one per-tensor
 * scale) or N; any K (K a multiple of 32 up to 16384 runs the streaming GEMV,
 * others the any-shape GEMV).
 */
TB_API int tb_w8a32_linear(const float *x, const int8_t *w, const float *scales, int64_t s_len,
                           const float *bias, float *out, int64_t m, int64_t n, int64_t k,
                           void *stream);

/*
 * INT8 SwiGLU MLP, fused_swiglu_mlp_w8a32 (binding src/ffi/quantization_ffi.rs:150-201,
 * kernel src/quantization/fused_ops.rs:8-133), with an optional residual add:
 *   h[j] = silu(dot(x, gate_j) * gs + gb[j]) * (dot(x, up_j) * us + ub[j]),
 *   out = dot(h, down_n) * ds + db[n] [+ residual].
 * Each projection's scales have *_s_len = 1 (one per-tensor scalar,
 * fused_ops.rs:80-97) or N (per row) elements; biases may be NULL; any K and
 * inter.  h [M, I] lives in the library workspace.
 */
TB_API int tb_fused_swiglu_mlp_w8a32(const float *x, const int8_t *gate_w, const float *gate_s,
                                     int64_t gate_s_len, const float *gate_b,
                                     const int8_t *up_w, const float *up_s, int64_t up_s_len,
                                     const float *up_b, const int8_t *down_w,
                                     const float *down_s, int64_t down_s_len,
                                     const float *down_b, const float *residual, float *out,
                                     int64_t m, int64_t k, int64_t inter, int64_t n_out,
                                     void *stream);

/* ------------------------------------------------------------------------ */
/* Decoder (replaces RustQwenDecoder, reference src/llm/decoder.rs:176-1374)   */
/*
 * Per-layer decode steps on caller-owned device buffers (one token, M = 1).
 *
 * fused_attention_step_w4a32 (binding src/ffi/quantization_ffi.rs:345-406,
 * kernel src/quantization/fused_ops.rs:891-1062):
 *   qkv = W_qkv x + qkv_b; RoPE on q and k with the current position's row
 *   cos / sin [head_dim] (q1' = q1 c[i] - q2 s[i], q2' = q2 c[i+d/2] + q1 s[i+d/2]);
 *   k, v appended to k_cache / v_cache [num_kv_heads, max_seq, head_dim] at
 *   `offset`; GQA attention over positions 0..offset; out = W_o attn + o_b.
 * The caches are updated in place, as the reference's are.  TB_UNSUPPORTED when
 * offset >= max_seq (the reference panics), when num_heads is not a multiple of
 * num_kv_heads, or for head_dim outside {32, 64, ..., 256}.
 */
TB_API int tb_fused_attention_step_w4a32(const float *x, const uint8_t *qkv_w, const float *qkv_s,
                                         const float *qkv_b, const uint8_t *o_w,
                                         const float *o_s, const float *o_b, float *k_cache,
                                         float *v_cache, const float *cos, const float *sin,
                                         float *out, int64_t hidden, int64_t offset,
                                         int64_t max_seq, int64_t num_heads,
                                         int64_t num_kv_heads, int64_t head_dim,
                                         int64_t group_size, void *stream);

/* fused_attention_step_w8a32 (binding src/ffi/quantization_ffi.rs:284-343, kernel
 * src/quantization/fused_ops.rs:718-888): as above with INT8 per-channel weights,
 * scales of 1 or N elements. */
TB_API int tb_fused_attention_step_w8a32(const float *x, const int8_t *qkv_w, const float *qkv_s,
                                         int64_t qkv_s_len, const float *qkv_b,
                                         const int8_t *o_w, const float *o_s, int64_t o_s_len,
                                         const float *o_b, float *k_cache, float *v_cache,
                                         const float *cos, const float *sin, float *out,
                                         int64_t hidden, int64_t offset, int64_t max_seq,
                                         int64_t num_heads, int64_t num_kv_heads,
                                         int64_t head_dim, void *stream);

/*
 * fused_transformer_layer_step_w4a32 (binding src/ffi/quantization_ffi.rs:408-480,
 * kernel src/quantization/fused_transformer.rs:16-376), x [hidden] updated in place:
 *   xn = RMSNorm(x, input_norm_w, eps); x += attention step of xn (as above);
 *   xn = RMSNorm(x, post_norm_w, eps);
 *   x += W_down (silu(W_gate xn + gate_b) * (W_up xn + up_b)) + down_b.
 */
TB_API int tb_fused_transformer_layer_step_w4a32(
    float *x, const float *input_norm_w, const uint8_t *qkv_w, const float *qkv_s,
    const float *qkv_b, const uint8_t *o_w, const float *o_s, const float *o_b,
    const float *post_norm_w, const uint8_t *gate_w, const float *gate_s, const float *gate_b,
    const uint8_t *up_w, const float *up_s, const float *up_b, const uint8_t *down_w,
    const float *down_s, const float *down_b, float *k_cache, float *v_cache, const float *cos,
    const float *sin, int64_t hidden, int64_t intermediate, int64_t offset, int64_t max_seq,
    int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t group_size, double eps,
    void *stream);

/* ------------------------------------------------------------------------ */

typedef struct tb_decoder tb_decoder;

/* Constructor arguments of RustQwenDecoder::new (decoder.rs:176-212), plus the
 * weight formats: weight_bits 4 = INT4 grouped projections (the reference's
 * native decoder), 8 = INT8 per-channel projections (the reference runs INT8
 * through its per-layer path, python/torchburn/llm/model.py:214-239, 334-344);
 * lm_head_bits 4, 8 or 32 (fp32 nn.Linear lm_head, model.py:499-500). */
typedef struct {
    int64_t num_layers, hidden_size, intermediate_size, num_heads, num_kv_heads, head_dim;
    int64_t vocab_size, group_size, max_seq_len;
    double rms_norm_eps, rope_theta;
    int32_t weight_bits, lm_head_bits;
} tb_decoder_config;

/* RustQwenDecoder::new (decoder.rs:193-424): validates the configuration
 * (TB_ERR_VALUE), copies the embedding table [V, H], final norm [H] and lm_head
 * (w, s; s unused for fp32) to the device, builds the f64 RoPE tables and a
 * zeroed KV cache [L][num_kv_heads, max_seq_len, head_dim].  Pointers may be
 * host or device memory. */
TB_API int tb_decoder_create(const tb_decoder_config *cfg, const float *embed,
                             const float *final_norm, const void *lm_head_w,
                             const float *lm_head_s, tb_decoder **out);

/* One layer, in the reference's capsule order (decoder.rs:260-308); qkv_b may be
 * NULL.  Every layer must be set once before the first step. */
TB_API int tb_decoder_set_layer(tb_decoder *d, int64_t layer, const float *in_norm,
                                const void *qkv_w, const float *qkv_s, const void *o_w,
                                const float *o_s, const float *post_norm, const void *gate_w,
                                const float *gate_s, const void *up_w, const float *up_s,
                                const void *down_w, const float *down_s, const float *qkv_b);

/* step_internal + decode_step (decoder.rs:729-750, 1051-1374): logits_out (host,
 * vocab_size floats) and argmax_out may be NULL.  An out-of-range token or
 * offset >= max_seq_len gives zeroed logits and changes nothing else. */
TB_API int tb_decoder_step(tb_decoder *d, int64_t token, int64_t offset, float *logits_out,
                           int64_t *argmax_out);

/* decode_and_sample (decoder.rs:752-777, 878-1020): repetition penalty over
 * `recent`, then greedy (temperature <= 0 or not finite, or top_k == 1) or
 * top-k / top-p sampling from the decoder's seeded generator, on the device
 * for any top_k (tb_sample_logits; draws numbered from the last
 * tb_decoder_set_seed); vocabularies past 262144 read the logits back and
 * sample on the host. */
TB_API int tb_decoder_decode_and_sample(tb_decoder *d, int64_t token, int64_t offset,
                                        float temperature, int64_t top_k,
                                        float repetition_penalty, const int64_t *recent,
                                        int64_t n_recent, float top_p, int64_t *token_out);

/* Greedy generate_loop (decoder.rs:788-832): tokens_out receives up to
 * max_new_tokens ids (the first is first_token); *seq_len_out = seq_len + n.
 * eos_token_id < 0 means none.  Without an EOS the steps run as device-driven
 * graph replays with no host round trip. */
TB_API int tb_decoder_generate(tb_decoder *d, int64_t first_token, int64_t seq_len,
                               int64_t max_new_tokens, int64_t eos_token_id,
                               int64_t *tokens_out, int64_t *n_out, int64_t *seq_len_out);

/* generate_loop with sampling (decoder.rs:788-832, window 859-876): the window
 * starts as the last 64 of recent_seed (n_seed ids, may be NULL when 0), each
 * step pushes its input token, applies the penalty over the window and samples
 * the next token.  The steps inside the cache run as replays of a graph whose
 * tail samples on the device (no logits read back; with an EOS token one
 * 4-byte read per step), for any top_k.  Greedy without a penalty is
 * tb_decoder_generate. */
TB_API int tb_decoder_generate_sampled(tb_decoder *d, int64_t first_token, int64_t seq_len,
                                       int64_t max_new_tokens, float temperature, int64_t top_k,
                                       float repetition_penalty, float top_p,
                                       int64_t eos_token_id, const int64_t *recent_seed,
                                       int64_t n_seed, int64_t *tokens_out, int64_t *n_out,
                                       int64_t *seq_len_out);

/* verify_tokens (decoder.rs:565-581): logits_out (host [n, vocab]) receives the
 * logits of every position start_offset + i, the KV cache gains the n rows.  An
 * INT4 decoder runs the n positions as one batched forward (the prefill path,
 * lm_head on every row); TB_ERR_VALUE when start_offset + n > max_seq_len. */
TB_API int tb_decoder_verify(tb_decoder *d, int64_t start_offset, const int64_t *tokens,
                             int64_t n, float *logits_out);

/* speculative_accept (decoder.rs:588-727): verify the k draft tokens at
 * `offset` (tb_decoder_verify), then Leviathan acceptance against draft_probs
 * (host [k, vocab] row-major) with the uniforms of the decoder's seeded stream
 * (tb_spec_uniform(seed, draw), draws continuing after tb_decoder_set_seed;
 * the reference seeds from the clock).  k == 0 gives (0, vocab - 1). */
TB_API int tb_decoder_speculative_accept(tb_decoder *d, int64_t offset,
                                         const int64_t *draft_tokens, int64_t k,
                                         const float *draft_probs, float temperature, float top_p,
                                         int64_t *accepted, int64_t *bonus);

/* The acceptance of speculative_accept over given target logits rows (host
 * [k, vocab]) and uniforms u[0..n_u) (at most k + 1 are used, in order). */
TB_API int tb_speculative_accept_rows(const float *target_rows, const int64_t *draft_tokens,
                                      const float *draft_probs, int64_t k, int64_t vocab,
                                      float temperature, float top_p, const double *u,
                                      int64_t n_u, int64_t *accepted, int64_t *bonus);

/* The f64 uniform in [0, 1) (53 bits) of draw `counter` under `seed`. */
TB_API double tb_spec_uniform(uint64_t seed, uint64_t counter);

/* prefill_tokens (decoder.rs:431-447): TB_ERR_VALUE when start_offset + n >
 * max_seq_len. */
TB_API int tb_decoder_prefill(tb_decoder *d, const int64_t *tokens, int64_t n,
                              int64_t start_offset, int64_t *offset_out);

/* reset_kv_cache / copy_kv_cache_from_tensors / kv_len / get_logits
 * (decoder.rs:449-533).  copy_kv sources are [num_kv_heads, src_max, head_dim]. */
TB_API int tb_decoder_reset_kv(tb_decoder *d);
TB_API int tb_decoder_copy_kv(tb_decoder *d, int64_t layer, const float *k, const float *v,
                              int64_t src_max, int64_t seq_len);
TB_API int tb_decoder_kv_len(tb_decoder *d, int64_t *out);
TB_API int tb_decoder_get_logits(tb_decoder *d, float *out);

/* Seed of the sampling generator (no reference counterpart: the reference draws
 * from an unseeded rand::random). */
TB_API int tb_decoder_set_seed(tb_decoder *d, uint64_t seed);

/* Replaces the RoPE tables, which tb_decoder_create builds in f64 as
 * RustQwenDecoder::new does (decoder.rs:334-350), with caller-built cos / sin
 * [max_seq_len, head_dim] (host or device memory).  The reference's per-layer
 * Python path, which runs INT8 and fp32-lm_head models, takes its tables from
 * RotaryEmbedding in f32 (python/torchburn/llm/model.py:108-122); no
 * counterpart on RustQwenDecoder. */
TB_API int tb_decoder_set_rope_tables(tb_decoder *d, const float *cos_t, const float *sin_t,
                                      int64_t rows, int64_t head_dim);

/* Attention length of a step: the step at position p scores positions
 * 0 .. min(p + 1, cap) - 1.  The default, 32768, is RustQwenDecoder's native
 * step, which caps its scores at the first 32768 positions
 * (src/llm/decoder.rs:1179-1184); cap 0 scores every position, as the
 * reference's per-layer Python path does (fused_ops.rs:997-1040).  Batched
 * prefill and verify chunks that reach the cap run step by step. */
TB_API int tb_decoder_set_attention_cap(tb_decoder *d, int64_t cap);

TB_API int tb_decoder_destroy(tb_decoder *d);

#ifdef __cplusplus
}
#endif

#endif /* TBHIP_H */

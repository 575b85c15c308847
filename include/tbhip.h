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
 * default stream); they are asynchronous on that stream and re-entrant per
 * stream.  The decoder copies HOST weights to the device once at creation, as
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
 * or NULL, out f32 [M, N].  group_size is 32 or 64 and must divide K.
 * M <= 15 runs the GEMV kernels; M >= 16 runs the dequantize + FP32-MFMA GEMM.
 */
TB_API int tb_w4a32_grouped_linear(const float *x, const uint8_t *w_packed, const float *scales,
                            const float *bias, float *out, int64_t m, int64_t n, int64_t k,
                            int64_t group_size, void *stream);

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

#ifdef __cplusplus
}
#endif

#endif /* TBHIP_H */

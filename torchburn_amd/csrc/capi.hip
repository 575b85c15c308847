// extern "C" entry points of libtbhip.so (declared in include/tbhip.h).
//
// Argument validation mirrors the reference's shape checks
// (src/quantization/packed_v2.rs:565-596) and returns TB_ERR_UNSUPPORTED with
// the reference's "TB_UNSUPPORTED:" marker, which the Python layer maps to
// UnsupportedOpError.
#include <math.h>
#include <stdlib.h>

#include <algorithm>
#include <atomic>

#include <mutex>
#include <string>
#include <vector>

#include "gemv_dense.hpp"
#include "tb_common.hpp"
#include "w4_gemv.hpp"
#include "w4_mfma.hpp"
#include "v2_layout.hpp"
#include "quantize.hpp"
#include "sample.hpp"

namespace tb {

namespace {
thread_local std::string g_last_error;

// Device workspace (grow-only, one per device) for intermediates of fused ops.
std::mutex g_ws_mu;
std::vector<std::pair<void *, size_t>> g_ws;

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int gshift_of(int64_t gs) { return gs == 32 ? 5 : (gs == 64 ? 6 : -1); }

// GEMV rows per block; TB_W4_J overrides the default (tuning sweeps only).
int env_int(const char *name, int dflt) {
    const char *e = getenv(name);
    int v = e ? atoi(e) : dflt;
    return v < 0 ? dflt : v;
}
int rows_j_env() {
    static int v = env_int("TB_W4_J", 0);
    return v;
}
// Activation rows from which INT4 projections run on FP32 MFMA instead of the
// GEMV (measured crossover: passes of 2 rows re-read the weights, the MFMA
// tile pads to 16 rows; TB_MFMA_MIN_M overrides, for tuning sweeps only).
int64_t mfma_min_m() {
    static int v = env_int("TB_MFMA_MIN_M", 5);
    return v < 1 ? 1 : v;
}
}  // namespace

int fail(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

int workspace(size_t bytes, void **out) {
    int dev = 0;
    TB_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_ws_mu);
    if ((int)g_ws.size() <= dev) g_ws.resize(dev + 1, {nullptr, 0});
    auto &slot = g_ws[dev];
    if (slot.second < bytes) {
        // A stream may still be using the old buffer; free it only after the
        // device is idle.
        if (slot.first) {
            TB_HIP(hipDeviceSynchronize());
            TB_HIP(hipFree(slot.first));
            slot = {nullptr, 0};
        }
        size_t sz = bytes < (1u << 20) ? (1u << 20) : bytes;
        TB_HIP(hipMalloc(&slot.first, sz));
        slot.second = sz;
    }
    *out = slot.first;
    return TB_OK;
}

// Validates a grouped INT4 projection and fills the common W4Params fields.
static int check_w4(const float *x, const uint8_t *w, const float *s, int64_t m, int64_t n,
                    int64_t k, int64_t gs, const char *what) {
    const std::string op(what);
    TB_REQUIRE(x && w && s, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: " + op + ": null pointer");
    TB_REQUIRE(m >= 0 && n >= 0 && k > 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": negative or empty dimension");
    TB_REQUIRE(gshift_of(gs) > 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": group_size must be 32 or 64, got " + std::to_string(gs));
    TB_REQUIRE(k % gs == 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": K=" + std::to_string(k) +
                   " must be a multiple of group_size=" + std::to_string(gs));
    TB_REQUIRE(k <= (1 << 20) && n < (1ll << 31) && m < (1ll << 31), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": dimension too large");
    TB_REQUIRE(aligned(x, 16) && aligned(w, 16) && aligned(s, 4), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": x and w must be 16-byte aligned device pointers");
    return TB_OK;
}

static W4Params w4_params(const float *x, const uint8_t *w, const float *s, const float *b,
                          float *y, int64_t m, int64_t n, int64_t k, int64_t gs) {
    W4Params p{};
    p.x = x; p.w0 = w; p.s0 = s; p.b0 = b; p.y = y;
    p.m = (int)m; p.n = (int)n; p.k = (int)k; p.gshift = gshift_of(gs);
    p.rows_j = rows_j_env();
    return p;
}

static MfmaParams mfma_params(const float *x, const uint8_t *w, const float *s, const float *b,
                              float *y, int64_t m, int64_t n, int64_t k, int64_t gs) {
    MfmaParams p{};
    p.x = x; p.w0 = w; p.s0 = s; p.b0 = b; p.y = y;
    p.m = (int)m; p.n = (int)n; p.k = (int)k; p.gshift = gshift_of(gs);
    return p;
}

// The MFMA projection with its split-K partials in the library workspace.
static int mfma_ws(const MfmaParams &p, int epi, hipStream_t st) {
    void *ws = nullptr;
    int rc = workspace(w4_mfma_partials_bytes(p.m, p.n, p.k, p.w1 != nullptr), &ws);
    if (rc) return rc;
    return w4_mfma(p, epi, static_cast<float *>(ws), st);
}

static size_t xq_bytes(int64_t m, int64_t k) {
    return (size_t)m * (size_t)(k / 32) * kXRecDwords * sizeof(uint32_t);
}

// M rows in passes of at most kMaxW4RowsPerPass (the GEMV keeps x in VGPRs).
// xq: chunk records of all m rows of p.x (built here when build_xq is set).
static int w4_rows(W4Params p, int epi, int64_t m, uint32_t *xq, bool build_xq,
                   hipStream_t st) {
    if (build_xq) {
        int rc = xquant(p.x, xq, (int)m, p.k, st);
        if (rc) return rc;
    }
    const int64_t rec = (int64_t)(p.k / 32) * kXRecDwords;
    for (int64_t r0 = 0; r0 < m; r0 += kMaxW4RowsPerPass) {
        W4Params q = p;
        q.m = (int)((m - r0) < kMaxW4RowsPerPass ? (m - r0) : kMaxW4RowsPerPass);
        q.x = p.x + r0 * p.k;
        q.xq = xq + r0 * rec;
        q.y = p.y + r0 * (int64_t)p.n;
        if (p.res) q.res = p.res + r0 * (int64_t)p.n;
        int rc = w4_gemv(q, epi, st);
        if (rc) return rc;
    }
    return TB_OK;
}

// W4A8 semantics of the reference's AVX-512 VNNI tier for group-64 INT4
// projections (gemv.rs:1392-1473, packed_v2.rs:366-370): off by default, the
// exact W4A32 contraction of its scalar / AVX2 / AVX-512 tiers.
std::atomic<int> g_vnni{0};

static size_t up256(size_t b) { return (b + 255) & ~(size_t)255; }

// One INT4 projection y = x . deq(W)^T (+ bias) (+ residual) over m rows, with
// the weights as v1 nibbles + f32 scales or as v2 blocks.  Under W4A8
// semantics (group 64) each row of x is first replaced by its byte
// quantization q * s_x.  Workspace: [x' | records or split-K partials].
static int linear_w4(const float *x, const uint8_t *w, const float *s, bool v2,
                     const float *bias, const float *res, float *out, int64_t m, int64_t n,
                     int64_t k, int64_t gs, hipStream_t st) {
    const bool a8 = gs == 64 && g_vnni.load(std::memory_order_relaxed) != 0;
    const size_t xb = a8 ? up256((size_t)m * (size_t)k * sizeof(float)) : 0;
    const int epi = res ? EPI_RESID : EPI_PLAIN;
    const bool mf = m >= mfma_min_m();
    const size_t rest = mf ? w4_mfma_partials_bytes((int)m, (int)n, (int)k, false)
                           : xq_bytes(m, k);
    void *ws = nullptr;
    int rc = workspace(xb + rest, &ws);
    if (rc) return rc;
    const float *xin = x;
    if (a8) {
        if ((rc = act_u8(x, static_cast<float *>(ws), m, k, st))) return rc;
        xin = static_cast<const float *>(ws);
    }
    void *tail = static_cast<char *>(ws) + xb;
    if (mf) {
        MfmaParams q = mfma_params(xin, w, s, bias, out, m, n, k, gs);
        q.res = res;
        q.v2 = v2 ? 1 : 0;
        return w4_mfma(q, epi, static_cast<float *>(tail), st);
    }
    W4Params p = w4_params(xin, w, s, bias, out, m, n, k, gs);
    p.res = res;
    p.v2 = v2 ? 1 : 0;
    return w4_rows(p, epi, m, static_cast<uint32_t *>(tail), true, st);
}

// Validates a v2 projection: group 64, K % 64 == 0, 4-byte aligned blocks.
static int check_v2(const float *x, const uint8_t *w, int64_t m, int64_t n, int64_t k,
                    int64_t gs, const char *what) {
    const std::string op(what);
    TB_REQUIRE(x && w, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: " + op + ": null pointer");
    TB_REQUIRE(m >= 0 && n >= 0 && k > 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": negative or empty dimension");
    TB_REQUIRE(gs == 64, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": the v2 layout is defined for 64-element groups, got " +
                   std::to_string(gs));
    TB_REQUIRE(k % 64 == 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": K=" + std::to_string(k) +
                   " must be a multiple of 64 for the v2 layout");
    TB_REQUIRE(k <= (1 << 20) && n < (1ll << 31) && m < (1ll << 31) &&
                   (size_t)n * (size_t)(k / 64) * 34 < (1ull << 32),
               TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: " + op + ": dimension too large");
    TB_REQUIRE(aligned(x, 16) && aligned(w, 4), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op +
                   ": x must be 16-byte and the blocks 4-byte aligned device pointers");
    return TB_OK;
}

static int check_w8(const float *x, const int8_t *w, const float *s, int64_t s_len, int64_t m,
                    int64_t n, int64_t k, const char *what) {
    const std::string op(what);
    TB_REQUIRE(x && w && s, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: " + op + ": null pointer");
    TB_REQUIRE(m >= 0 && n >= 0 && k > 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": negative or empty dimension");
    TB_REQUIRE(s_len == 1 || s_len == n, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": scales must have 1 or N elements");
    TB_REQUIRE(k % 32 == 0 && k <= (1 << 20) && n < (1ll << 31), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": K must be a multiple of 32");
    TB_REQUIRE(aligned(x, 16) && aligned(w, 16), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": x and w must be 16-byte aligned device pointers");
    return TB_OK;
}

static int dense_rows(DenseParams p, int wt, int epi, int64_t m, hipStream_t st) {
    for (int64_t r0 = 0; r0 < m; r0 += kMaxRowsPerPass) {
        DenseParams q = p;
        q.m = (int)((m - r0) < kMaxRowsPerPass ? (m - r0) : kMaxRowsPerPass);
        q.x = p.x + r0 * p.k;
        q.y = p.y + r0 * (int64_t)p.n;
        if (p.res) q.res = p.res + r0 * (int64_t)p.n;
        int rc = dense_gemv(q, wt, epi, st);
        if (rc) return rc;
    }
    return TB_OK;
}

}  // namespace tb

using namespace tb;

extern "C" {

const char *tb_last_error(void) { return g_last_error.c_str(); }

const char *tb_version(void) { return "torchburn_amd 0.1.0 gfx950"; }

int tb_w4a32_grouped_linear(const float *x, const uint8_t *w_packed, const float *scales,
                            const float *bias, float *out, int64_t m, int64_t n, int64_t k,
                            int64_t group_size, void *stream) {
    int rc = check_w4(x, w_packed, scales, m, n, k, group_size, "w4a32_grouped_linear");
    if (rc) return rc;
    TB_REQUIRE(out, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: w4a32_grouped_linear: null output");
    if (m == 0 || n == 0) return TB_OK;
    return linear_w4(x, w_packed, scales, false, bias, nullptr, out, m, n, k, group_size,
                     (hipStream_t)stream);
}

int tb_w4a32_grouped_linear_v2(const float *x, const uint8_t *w_blocked, const float *bias,
                               float *out, int64_t m, int64_t n, int64_t k, int64_t group_size,
                               void *stream) {
    int rc = check_v2(x, w_blocked, m, n, k, group_size, "w4a32_grouped_linear_v2");
    if (rc) return rc;
    TB_REQUIRE(out, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: w4a32_grouped_linear_v2: null output");
    if (m == 0 || n == 0) return TB_OK;
    return linear_w4(x, w_blocked, nullptr, true, bias, nullptr, out, m, n, k, 64,
                     (hipStream_t)stream);
}

int tb_pack_rows_w4a32_group64_v1_to_v2(const uint8_t *w_packed, const float *scales,
                                        uint8_t *out, int64_t n, int64_t k, void *stream) {
    TB_REQUIRE(w_packed && scales && out, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: pack_rows_w4a32_group64_v1_to_v2: null pointer");
    TB_REQUIRE(n >= 0 && k > 0 && k % 64 == 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: pack_rows_w4a32_group64_v1_to_v2: K=" + std::to_string(k) +
                   " must be a positive multiple of 64");
    TB_REQUIRE(aligned(w_packed, 16) && aligned(scales, 4) && aligned(out, 2), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: pack_rows_w4a32_group64_v1_to_v2: misaligned device pointer");
    return pack_v1_to_v2(w_packed, scales, out, n, k, (hipStream_t)stream);
}

int tb_dequantize_int4_grouped_v2(const uint8_t *w_blocked, float *out, int64_t n, int64_t k,
                                  void *stream) {
    TB_REQUIRE(w_blocked && out, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: dequantize_int4_grouped_v2: null pointer");
    TB_REQUIRE(n >= 0 && k > 0 && k % 64 == 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: dequantize_int4_grouped_v2: K=" + std::to_string(k) +
                   " must be a positive multiple of 64");
    TB_REQUIRE(aligned(w_blocked, 4) && aligned(out, 16), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: dequantize_int4_grouped_v2: misaligned device pointer");
    TB_REQUIRE((size_t)n * (size_t)(k / 64) * 34 < (1ull << 32), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: dequantize_int4_grouped_v2: blocks must be under 4 GiB");
    return dequant_v2(w_blocked, out, n, k, (hipStream_t)stream);
}

int tb_quantize_weight_int4_grouped(const float *w, uint8_t *packed, float *scales, int64_t n,
                                    int64_t k, int64_t group_size, void *stream) {
    TB_REQUIRE(w && packed && scales, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: quantize_weight_int4_grouped: null pointer");
    TB_REQUIRE(group_size == 32 || group_size == 64, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: quantize_weight_int4_grouped: group_size must be 32 or 64, got " +
                   std::to_string(group_size));
    TB_REQUIRE(n >= 0 && k > 0 && k <= (1 << 30), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: quantize_weight_int4_grouped: bad shape");
    TB_REQUIRE(k % group_size == 0, TB_ERR_VALUE,
               "Weight dimension K=" + std::to_string(k) + " must be divisible by group_size=" +
                   std::to_string(group_size) + ". Consider padding the weight tensor along dim 1 "
                   "to a multiple of " + std::to_string(group_size) + ".");
    TB_REQUIRE(aligned(w, 4) && aligned(scales, 4), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: quantize_weight_int4_grouped: misaligned device pointer");
    return quantize_int4_grouped(w, packed, scales, n, k, (int)group_size, (hipStream_t)stream);
}

int tb_quantize_weight_int8(const float *w, int8_t *q, float *scales, int64_t n, int64_t k,
                            void *stream) {
    TB_REQUIRE(w && q && scales, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: quantize_weight_int8: null pointer");
    TB_REQUIRE(n >= 0 && k > 0 && k <= (1 << 30) && n < (1ll << 31), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: quantize_weight_int8: bad shape");
    TB_REQUIRE(aligned(w, 4) && aligned(scales, 4), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: quantize_weight_int8: misaligned device pointer");
    return quantize_int8(w, q, scales, n, k, (hipStream_t)stream);
}

int tb_unpack_rows_w4a32_group64_v2_to_v1(const uint8_t *w_blocked, uint8_t *w_packed,
                                          float *scales, int64_t n, int64_t k, void *stream) {
    TB_REQUIRE(w_blocked && w_packed && scales, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: unpack_rows_w4a32_group64_v2_to_v1: null pointer");
    TB_REQUIRE(n >= 0 && k > 0 && k % 64 == 0 && (size_t)n * (size_t)(k / 64) * 34 < (1ull << 32),
               TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: unpack_rows_w4a32_group64_v2_to_v1: K must be a multiple of 64 "
               "and the blocks under 4 GiB");
    TB_REQUIRE(aligned(w_blocked, 4) && aligned(w_packed, 16) && aligned(scales, 4),
               TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: unpack_rows_w4a32_group64_v2_to_v1: misaligned device pointer");
    return unpack_v2_to_v1(w_blocked, w_packed, scales, n, k, (hipStream_t)stream);
}

float tb_sample_uniform(uint64_t seed, uint64_t counter) { return sample_uniform(seed, counter); }

int tb_sample_logits(float *logits, int64_t vocab, float temperature, int64_t top_k, float top_p,
                     float repetition_penalty, const int64_t *recent, int64_t n_recent,
                     uint64_t seed, uint64_t counter, int64_t *token_out, float *u_out,
                     void *stream) {
    TB_REQUIRE(logits && token_out, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: sample_logits: null pointer");
    TB_REQUIRE(vocab > 0 && vocab <= (int64_t)kSampleMaxBlocks * kSampleSlice, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: sample_logits: vocabulary of " + std::to_string(vocab) +
                   " outside 1.." + std::to_string(kSampleMaxBlocks * kSampleSlice));
    TB_REQUIRE(n_recent <= 0 || recent, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: sample_logits: null recent tokens");
    // decoder.rs:919-931: greedy when the temperature is not usable or top_k == 1
    const bool greedy = !std::isfinite(temperature) || temperature <= 0.f || top_k == 1;
    const int64_t k = greedy ? 1 : std::max<int64_t>(1, std::min<int64_t>(top_k, vocab));
    TB_REQUIRE(k <= kSampleMaxK, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: device sampling takes top_k <= " + std::to_string(kSampleMaxK));
    SampleParams prm{};
    prm.temperature = temperature;
    prm.top_p = top_p;
    prm.penalty = repetition_penalty;
    prm.k = (int)k;
    prm.greedy = greedy ? 1 : 0;
    prm.seed = seed;
    prm.counter = counter;
    const size_t cand = (size_t)kSampleCand;
    const size_t bytes = up256(sizeof(SampleParams)) + up256(sizeof(SampleOut)) +
                         up256(cand * 4) + up256(cand * 4) + up256(kSampleMaxBlocks * 4);
    void *ws = nullptr;
    int rc = workspace(bytes, &ws);
    if (rc) return rc;
    char *w = static_cast<char *>(ws);
    SampleParams *dprm = reinterpret_cast<SampleParams *>(w);
    w += up256(sizeof(SampleParams));
    SampleOut *dout = reinterpret_cast<SampleOut *>(w);
    w += up256(sizeof(SampleOut));
    SampleScratch sc;
    sc.key = reinterpret_cast<uint32_t *>(w);
    w += up256(cand * 4);
    sc.idx = reinterpret_cast<int *>(w);
    w += up256(cand * 4);
    sc.cnt = reinterpret_cast<int *>(w);
    hipStream_t st = (hipStream_t)stream;
    TB_HIP(hipMemcpyAsync(dprm, &prm, sizeof(prm), hipMemcpyHostToDevice, st));
    rc = launch_sample(logits, (int)vocab, recent, (int)n_recent, dprm, sc, dout, st);
    if (rc) return rc;
    SampleOut ho{};
    TB_HIP(hipMemcpyAsync(&ho, dout, sizeof(ho), hipMemcpyDeviceToHost, st));
    TB_HIP(hipStreamSynchronize(st));
    *token_out = ho.token;
    if (u_out) *u_out = ho.u;
    return TB_OK;
}

int tb_set_vnni_semantics(int enabled) {
    return g_vnni.exchange(enabled ? 1 : 0);
}

int tb_w4a32_grouped_linear_residual(const float *x, const uint8_t *w_packed,
                                     const float *scales, const float *bias,
                                     const float *residual, float *out, int64_t m, int64_t n,
                                     int64_t k, int64_t group_size, void *stream) {
    int rc = check_w4(x, w_packed, scales, m, n, k, group_size, "w4a32_grouped_linear_residual");
    if (rc) return rc;
    TB_REQUIRE(out && residual, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: w4a32_grouped_linear_residual: null output or residual");
    if (m == 0 || n == 0) return TB_OK;
    return linear_w4(x, w_packed, scales, false, bias, residual, out, m, n, k, group_size,
                     (hipStream_t)stream);
}

int tb_swiglu_w4a32(const float *x, const uint8_t *gate_w, const float *gate_s,
                    const float *gate_b, const uint8_t *up_w, const float *up_s,
                    const float *up_b, float *h, int64_t m, int64_t k, int64_t inter,
                    int64_t group_size, void *stream) {
    int rc = check_w4(x, gate_w, gate_s, m, inter, k, group_size, "swiglu_w4a32");
    if (rc) return rc;
    rc = check_w4(x, up_w, up_s, m, inter, k, group_size, "swiglu_w4a32");
    if (rc) return rc;
    TB_REQUIRE(h, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: swiglu_w4a32: null output");
    if (m == 0 || inter == 0) return TB_OK;
    if (m >= mfma_min_m()) {
        MfmaParams q = mfma_params(x, gate_w, gate_s, gate_b, h, m, inter, k, group_size);
        q.w1 = up_w; q.s1 = up_s; q.b1 = up_b;
        return mfma_ws(q, EPI_SWIGLU, (hipStream_t)stream);
    }
    void *ws = nullptr;
    rc = workspace(xq_bytes(m, k), &ws);
    if (rc) return rc;
    W4Params p = w4_params(x, gate_w, gate_s, gate_b, h, m, inter, k, group_size);
    p.w1 = up_w; p.s1 = up_s; p.b1 = up_b;
    return w4_rows(p, EPI_SWIGLU, m, (uint32_t *)ws, true, (hipStream_t)stream);
}

int tb_fused_swiglu_mlp_w4a32(const float *x, const uint8_t *gate_w, const float *gate_s,
                              const float *gate_b, const uint8_t *up_w, const float *up_s,
                              const float *up_b, const uint8_t *down_w, const float *down_s,
                              const float *down_b, const float *residual, float *out,
                              int64_t m, int64_t k, int64_t inter, int64_t n_out,
                              int64_t group_size, void *stream) {
    int rc = check_w4(x, gate_w, gate_s, m, inter, k, group_size, "fused_swiglu_mlp_w4a32");
    if (rc) return rc;
    rc = check_w4(x, up_w, up_s, m, inter, k, group_size, "fused_swiglu_mlp_w4a32");
    if (rc) return rc;
    TB_REQUIRE(inter % group_size == 0 && inter % 32 == 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: fused_swiglu_mlp_w4a32: intermediate size must be a multiple "
               "of group_size");
    TB_REQUIRE(down_w && down_s && out, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: fused_swiglu_mlp_w4a32: null down weight or output");
    if (m == 0 || n_out == 0) return TB_OK;
    // Workspace: h [m, inter] f32 | chunk records of x | chunk records of h,
    // or on the MFMA path h | split-K partials.
    const size_t hb = ((size_t)m * (size_t)inter * sizeof(float) + 255) & ~(size_t)255;
    if (m >= mfma_min_m()) {
        const size_t pg = w4_mfma_partials_bytes((int)m, (int)inter, (int)k, true);
        const size_t pd = w4_mfma_partials_bytes((int)m, (int)n_out, (int)inter, false);
        void *ws = nullptr;
        rc = workspace(hb + (pg > pd ? pg : pd), &ws);
        if (rc) return rc;
        float *h = static_cast<float *>(ws);
        float *part = reinterpret_cast<float *>(static_cast<char *>(ws) + hb);
        hipStream_t st = (hipStream_t)stream;
        MfmaParams g = mfma_params(x, gate_w, gate_s, gate_b, h, m, inter, k, group_size);
        g.w1 = up_w; g.s1 = up_s; g.b1 = up_b;
        rc = w4_mfma(g, EPI_SWIGLU, part, st);
        if (rc) return rc;
        MfmaParams d = mfma_params(h, down_w, down_s, down_b, out, m, n_out, inter, group_size);
        d.res = residual;
        return w4_mfma(d, residual ? EPI_RESID : EPI_PLAIN, part, st);
    }
    const size_t xb = (xq_bytes(m, k) + 255) & ~(size_t)255;
    void *ws = nullptr;
    rc = workspace(hb + xb + xq_bytes(m, inter), &ws);
    if (rc) return rc;
    float *h = static_cast<float *>(ws);
    uint32_t *xq = reinterpret_cast<uint32_t *>(static_cast<char *>(ws) + hb);
    uint32_t *hq = reinterpret_cast<uint32_t *>(static_cast<char *>(ws) + hb + xb);
    hipStream_t st = (hipStream_t)stream;
    W4Params p = w4_params(x, gate_w, gate_s, gate_b, h, m, inter, k, group_size);
    p.w1 = up_w; p.s1 = up_s; p.b1 = up_b;
    if (m == 1) {
        // One row: the gate/up epilogue writes h's chunk records as well, so the
        // down projection needs no separate record pass.
        rc = xquant(x, xq, 1, (int)k, st);
        if (rc) return rc;
        p.xq = xq;
        p.rec_out = hq;
        rc = w4_gemv(p, EPI_SWIGLU, st);
        if (rc) return rc;
        W4Params d = w4_params(h, down_w, down_s, down_b, out, m, n_out, inter, group_size);
        d.xq = hq;
        d.res = residual;
        return w4_gemv(d, residual ? EPI_RESID : EPI_PLAIN, st);
    }
    rc = w4_rows(p, EPI_SWIGLU, m, xq, true, st);
    if (rc) return rc;
    W4Params d = w4_params(h, down_w, down_s, down_b, out, m, n_out, inter, group_size);
    if (residual) {
        d.res = residual;
        return w4_rows(d, EPI_RESID, m, hq, true, st);
    }
    return w4_rows(d, EPI_PLAIN, m, hq, true, st);
}

int64_t tb_x_records_bytes(int64_t m, int64_t k) {
    return (m < 0 || k < 0) ? 0 : (int64_t)xq_bytes(m, k);
}

int tb_xquant(const float *x, uint32_t *xq, int64_t m, int64_t k, void *stream) {
    TB_REQUIRE(x && xq, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: xquant: null pointer");
    TB_REQUIRE(m >= 0 && k > 0 && k % 32 == 0 && k <= (1 << 20) && m < (1 << 24),
               TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: xquant: K must be a positive multiple of 32");
    TB_REQUIRE(aligned(x, 16) && aligned(xq, 16), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: xquant: 16-byte aligned device pointers required");
    return xquant(x, xq, (int)m, (int)k, (hipStream_t)stream);
}

int tb_w4a32_gemv_xq(const float *x, const uint32_t *xq, const uint8_t *w_packed,
                     const float *scales, const float *bias, const float *residual, float *out,
                     int64_t m, int64_t n, int64_t k, int64_t group_size, void *stream) {
    int rc = check_w4(x, w_packed, scales, m, n, k, group_size, "w4a32_gemv_xq");
    if (rc) return rc;
    TB_REQUIRE(out && xq && aligned(xq, 16), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: w4a32_gemv_xq: null output or unaligned records");
    if (m == 0 || n == 0) return TB_OK;
    if (m >= mfma_min_m()) {
        MfmaParams q = mfma_params(x, w_packed, scales, bias, out, m, n, k, group_size);
        q.res = residual;
        return mfma_ws(q, residual ? EPI_RESID : EPI_PLAIN, (hipStream_t)stream);
    }
    W4Params p = w4_params(x, w_packed, scales, bias, out, m, n, k, group_size);
    p.res = residual;
    return w4_rows(p, residual ? EPI_RESID : EPI_PLAIN, m, const_cast<uint32_t *>(xq), false,
                   (hipStream_t)stream);
}

int tb_swiglu_w4a32_xq(const float *x, const uint32_t *xq, const uint8_t *gate_w,
                       const float *gate_s, const float *gate_b, const uint8_t *up_w,
                       const float *up_s, const float *up_b, float *h, int64_t m, int64_t k,
                       int64_t inter, int64_t group_size, void *stream) {
    int rc = check_w4(x, gate_w, gate_s, m, inter, k, group_size, "swiglu_w4a32_xq");
    if (rc) return rc;
    rc = check_w4(x, up_w, up_s, m, inter, k, group_size, "swiglu_w4a32_xq");
    if (rc) return rc;
    TB_REQUIRE(h && xq && aligned(xq, 16), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: swiglu_w4a32_xq: null output or unaligned records");
    if (m == 0 || inter == 0) return TB_OK;
    if (m >= mfma_min_m()) {
        MfmaParams q = mfma_params(x, gate_w, gate_s, gate_b, h, m, inter, k, group_size);
        q.w1 = up_w; q.s1 = up_s; q.b1 = up_b;
        return mfma_ws(q, EPI_SWIGLU, (hipStream_t)stream);
    }
    W4Params p = w4_params(x, gate_w, gate_s, gate_b, h, m, inter, k, group_size);
    p.w1 = up_w; p.s1 = up_s; p.b1 = up_b;
    return w4_rows(p, EPI_SWIGLU, m, const_cast<uint32_t *>(xq), false, (hipStream_t)stream);
}

int tb_w8a32_linear(const float *x, const int8_t *w, const float *scales, int64_t s_len,
                    const float *bias, float *out, int64_t m, int64_t n, int64_t k,
                    void *stream) {
    int rc = check_w8(x, w, scales, s_len, m, n, k, "w8a32_linear");
    if (rc) return rc;
    TB_REQUIRE(out, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: w8a32_linear: null output");
    if (m == 0 || n == 0) return TB_OK;
    DenseParams p{};
    p.x = x; p.w0 = w; p.rs0 = scales; p.rs0_len = (int)s_len; p.b0 = bias; p.y = out;
    p.m = (int)m; p.n = (int)n; p.k = (int)k;
    return dense_rows(p, W_I8, EPI_PLAIN, m, (hipStream_t)stream);
}

int tb_fused_swiglu_mlp_w8a32(const float *x, const int8_t *gate_w, const float *gate_s,
                              const float *gate_b, const int8_t *up_w, const float *up_s,
                              const float *up_b, const int8_t *down_w, const float *down_s,
                              const float *down_b, const float *residual, float *out,
                              int64_t m, int64_t k, int64_t inter, int64_t n_out,
                              void *stream) {
    int rc = check_w8(x, gate_w, gate_s, inter, m, inter, k, "fused_swiglu_mlp_w8a32");
    if (rc) return rc;
    rc = check_w8(x, up_w, up_s, inter, m, inter, k, "fused_swiglu_mlp_w8a32");
    if (rc) return rc;
    TB_REQUIRE(down_w && down_s && out && inter % 32 == 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: fused_swiglu_mlp_w8a32: bad down projection or output");
    if (m == 0 || n_out == 0) return TB_OK;
    void *ws = nullptr;
    rc = workspace((size_t)m * (size_t)inter * sizeof(float), &ws);
    if (rc) return rc;
    float *h = static_cast<float *>(ws);
    hipStream_t st = (hipStream_t)stream;
    DenseParams p{};
    p.x = x; p.w0 = gate_w; p.rs0 = gate_s; p.rs0_len = (int)inter; p.b0 = gate_b;
    p.w1 = up_w; p.rs1 = up_s; p.rs1_len = (int)inter; p.b1 = up_b;
    p.y = h; p.m = (int)m; p.n = (int)inter; p.k = (int)k;
    rc = dense_rows(p, W_I8, EPI_SWIGLU, m, st);
    if (rc) return rc;
    DenseParams d{};
    d.x = h; d.w0 = down_w; d.rs0 = down_s; d.rs0_len = (int)n_out; d.b0 = down_b;
    d.res = residual; d.y = out; d.m = (int)m; d.n = (int)n_out; d.k = (int)inter;
    return dense_rows(d, W_I8, residual ? EPI_RESID : EPI_PLAIN, m, st);
}

}  // extern "C"

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

#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "gemv_dense.hpp"
#include "gemv_generic.hpp"
#include "tb_common.hpp"
#include "w4_gemv.hpp"
#include "w4_limb.hpp"
#include "w4_mfma.hpp"
#include "v2_layout.hpp"
#include "quantize.hpp"
#include "sample.hpp"

namespace tb {

namespace {
thread_local std::string g_last_error;

// Per-(device, stream) scratch for intermediates of the stateless ops.
struct StreamScratch {
    std::mutex mu;        // held by the op enqueueing on this stream
    void *ptr = nullptr;
    size_t size = 0;
    // buffers this workspace outgrew: a graph captured earlier may still read
    // them, so they are kept until tb_release_stream_workspace or process exit
    std::vector<void *> retired;
};
std::mutex g_ws_mu;       // guards g_ws
std::map<std::pair<int, uintptr_t>, std::unique_ptr<StreamScratch>> g_ws;

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// log2 of a power-of-two group size of at least 32 (the streaming kernels'
// chunk), else -1.
int gshift_of(int64_t gs) {
    if (gs < 32 || gs > (1 << 20) || (gs & (gs - 1)) != 0) return -1;
    int b = 0;
    while ((1ll << b) < gs) ++b;
    return b;
}

// K range of one GEMV pass (kMaxWaves K-slices of 64 chunks of 32 elements).
constexpr int64_t kMaxGemvK = 8 * 64 * 32;

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
// Batches of the small-batch f16-MFMA projection (w4_limb.hip), which reads
// the weights once for 3..16 activation rows (at 2 rows the two-row GEMV
// pass is faster: 41 vs 54 us for a Llama-3-8B MLP); TB_LIMB_MIN_M /
// TB_LIMB_MAX_M override (max 1 turns it off), for tuning sweeps only.
int64_t limb_min_m() {
    static int v = env_int("TB_LIMB_MIN_M", 3);
    return std::max(v, 2);
}
int64_t limb_max_m() {
    static int v = env_int("TB_LIMB_MAX_M", kLimbMaxM);
    return std::min<int64_t>(v, kLimbMaxM);
}
}  // namespace

int fail(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

int workspace(size_t bytes, hipStream_t st, WsLease &out) {
    int dev = 0;
    TB_HIP(hipGetDevice(&dev));
    StreamScratch *sc;
    {
        std::lock_guard<std::mutex> lk(g_ws_mu);
        auto &slot = g_ws[{dev, reinterpret_cast<uintptr_t>(st)}];
        if (!slot) slot.reset(new StreamScratch);
        sc = slot.get();
    }
    out.lock = std::unique_lock<std::mutex>(sc->mu);
    if (sc->size < bytes) {
        size_t sz = std::max<size_t>({bytes, 2 * sc->size, (size_t)1 << 20});
        void *p = nullptr;
        // A stream first seen under graph capture (e.g. a capture stream that
        // was never warmed up) allocates here: hipMalloc is not a stream
        // operation, so this thread's capture mode is relaxed around it.
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        TB_HIP(hipThreadExchangeStreamCaptureMode(&mode));
        const hipError_t e = hipMalloc(&p, sz);
        TB_HIP(hipThreadExchangeStreamCaptureMode(&mode));
        TB_HIP(e);
        if (sc->ptr) sc->retired.push_back(sc->ptr);
        sc->ptr = p;
        sc->size = sz;
    }
    out.ptr = sc->ptr;
    return TB_OK;
}

// Validates a grouped INT4 projection: any K >= 1 and any group size >= 1 (the
// reference's GEMV takes tail groups, src/quantization/gemv.rs:1650-1660).
static int check_w4(const float *x, const uint8_t *w, const float *s, int64_t m, int64_t n,
                    int64_t k, int64_t gs, const char *what) {
    const std::string op(what);
    TB_REQUIRE(x && w && s, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: " + op + ": null pointer");
    TB_REQUIRE(m >= 0 && n >= 0 && k > 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": negative or empty dimension");
    // Groups start on byte boundaries (gemv.rs:1514-1530 steps group_size / 2
    // bytes per group), so an odd group size has no consistent layout.
    TB_REQUIRE(gs >= 2 && gs % 2 == 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": group_size must be a positive even number, got " +
                   std::to_string(gs));
    TB_REQUIRE(k <= (1 << 30) && n < (1ll << 31) && m < (1ll << 31), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": dimension too large");
    TB_REQUIRE(aligned(x, 4) && aligned(s, 4), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": x and scales must be 4-byte aligned device pointers");
    return TB_OK;
}

// Shapes the streaming kernels take: K a multiple of 32 and of a power-of-two
// group of at least 32, 16-byte aligned x and w, and (GEMV passes, M below the
// MFMA threshold) K within one pass's split-K range.  Other shapes run the
// any-shape GEMV (gemv_generic.hip).
static bool w4_fast(const float *x, const void *w, int64_t m, int64_t k, int64_t gs,
                    bool per_row) {
    if (k % 32 != 0 || (!per_row && (gshift_of(gs) < 0 || k % gs != 0))) return false;
    if (!aligned(x, 16) || !aligned(w, 16)) return false;
    return m >= mfma_min_m() || k <= kMaxGemvK;
}

static W4Params w4_params(const float *x, const uint8_t *w, const float *s, const float *b,
                          float *y, int64_t m, int64_t n, int64_t k, int64_t gs) {
    W4Params p{};
    p.x = x; p.w0 = w; p.s0 = s; p.b0 = b; p.y = y;
    p.m = (int)m; p.n = (int)n; p.k = (int)k; p.gshift = std::max(gshift_of(gs), 5);
    p.rows_j = rows_j_env();
    return p;
}

static MfmaParams mfma_params(const float *x, const uint8_t *w, const float *s, const float *b,
                              float *y, int64_t m, int64_t n, int64_t k, int64_t gs) {
    MfmaParams p{};
    p.x = x; p.w0 = w; p.s0 = s; p.b0 = b; p.y = y;
    p.m = (int)m; p.n = (int)n; p.k = (int)k; p.gshift = std::max(gshift_of(gs), 5);
    return p;
}

// The MFMA projection with its split-K partials in the library workspace.
static int mfma_ws(const MfmaParams &p, int epi, hipStream_t st) {
    WsLease lease;
    int rc = workspace(w4_mfma_partials_bytes(p.m, p.n, p.k, p.w1 != nullptr), st, lease);
    if (rc) return rc;
    void *ws = lease.ptr;
    return w4_mfma(p, epi, static_cast<float *>(ws), st);
}

// Shapes of the small-batch f16-MFMA projection: limb_min_m() <= m <= limb_max_m(),
// K % 128 == 0 (a SwiGLU pair: N % 128 == 0), 16-byte aligned x and w, a power-of-two
// group >= 32 dividing K (or per-row / scalar scales).
static bool limb_fast(const float *x, const void *w, int64_t m, int64_t n, int64_t k,
                      int64_t gs, bool per_row, bool pair) {
    if (m < limb_min_m() || m > limb_max_m() || !limb_shape_ok(m, n, k, pair)) return false;
    if (!per_row && (gshift_of(gs) < 0 || k % gs != 0)) return false;
    return aligned(x, 16) && aligned(w, 16);
}

// scale_mode 0: grouped scales [n, k / gs]; 1: one per row; 2: one scalar.
static LimbParams limb_params(const float *x, const uint8_t *rec, const uint8_t *w,
                              const float *s, const float *b, float *y, int64_t m, int64_t n,
                              int64_t k, int64_t gs, int scale_mode = 0) {
    LimbParams p{};
    p.x = x; p.rec = rec; p.w0 = w; p.s0 = s; p.b0 = b; p.y = y;
    p.m = (int)m; p.n = (int)n; p.k = (int)k;
    p.scols = scale_mode == 0 ? (int)(k / gs) : (scale_mode == 1 ? 1 : 0);
    p.gshift = scale_mode == 0 ? gshift_of(gs) : 31;
    return p;
}

static size_t xq_bytes(int64_t m, int64_t k) {
    return (size_t)m * (size_t)(k / 32) * kXRecDwords * sizeof(uint32_t);
}

// M rows in passes of at most kMaxW4RowsPerPass (the GEMV keeps x in VGPRs).
// xq: chunk records of all m rows of p.x (built here when build_xq is set).  A
// single row of a single projection builds them inside the GEMV instead, one
// chunk per lane while its weights load (Qwen2.5-0.5B up-projection
// [4864, 896]: 7.0 -> 6.0 us); a gate/up pair keeps the record pass, since
// the build lengthens each of its two rounds of blocks (Llama-3-8B: +4 us
// against the pass's 2-4 us).
static int w4_rows(W4Params p, int epi, int64_t m, uint32_t *xq, bool build_xq,
                   hipStream_t st) {
    if (build_xq && m == 1 && p.w1 == nullptr && epi != EPI_ROPE && p.ssq_in == nullptr) {
        p.xq = nullptr;
        return w4_gemv(p, epi, st);
    }
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

bool vnni_semantics() { return g_vnni.load(std::memory_order_relaxed) != 0; }

static size_t up256(size_t b) { return (b + 255) & ~(size_t)255; }

// One INT4 projection y = x . deq(W)^T (+ bias) (+ residual) over m rows, with
// the weights as v1 nibbles + f32 scales or as v2 blocks.  Under W4A8
// semantics (group 64) each row of x is first replaced by its byte
// quantization q * s_x.  Workspace: [x' | records or split-K partials].
static int generic(const float *x, const void *w0, const float *s0, int mode0, const float *b0,
                   const void *w1, const float *s1, int mode1, const float *b1,
                   const float *res, float *y, int64_t m, int64_t n, int64_t k, int64_t gs,
                   int bits, hipStream_t st);

static int linear_w4(const float *x, const uint8_t *w, const float *s, bool v2,
                     const float *bias, const float *res, float *out, int64_t m, int64_t n,
                     int64_t k, int64_t gs, hipStream_t st, int scale_mode = 0) {
    // M = 16 with N and K at most 4096 takes the FP32-MFMA projection: all 16
    // rows share one LDS tile there, where the two-tile limb form needs five K
    // splits (14.4 against 15.4 us at N = K = 4096; from N = 14336 the limb
    // form is faster, 25.7 against 30.2 us)
    const bool lb = !v2 && limb_fast(x, w, m, n, k, gs, scale_mode != 0, false) &&
                    !(m == 16 && n <= 4096 && k <= 4096);
    const bool any_shape = !v2 && !lb && !w4_fast(x, w, m, k, gs, scale_mode != 0);
    // W4A8 applies to every group-64 projection, whichever kernel takes the
    // shape (gemv.rs:1559-1563).  With K % 64 != 0 the reference's VNNI row
    // reads its last group past the row and the activation bytes (undefined);
    // here the missing elements of that group count as zero.
    const bool a8 = gs == 64 && scale_mode == 0 && g_vnni.load(std::memory_order_relaxed) != 0;
    const size_t xb = a8 ? up256((size_t)m * (size_t)k * sizeof(float)) : 0;
    const int epi = res ? EPI_RESID : EPI_PLAIN;
    const bool mf = !lb && !any_shape && m >= mfma_min_m();
    const size_t rest = any_shape ? 0
                        : lb ? up256(limb_records_bytes((int)m, (int)k)) +
                                   limb_partials_bytes((int)m, (int)n, (int)k, false)
                        : mf ? w4_mfma_partials_bytes((int)m, (int)n, (int)k, false)
                             : xq_bytes(m, k);
    const float *xin = x;
    void *tail = nullptr;
    int rc;
    WsLease lease;
    if (xb + rest) {
        if ((rc = workspace(xb + rest, st, lease))) return rc;
        void *ws = lease.ptr;
        if (a8) {
            if ((rc = act_u8(x, static_cast<float *>(ws), m, k, st))) return rc;
            xin = static_cast<const float *>(ws);
        }
        tail = static_cast<char *>(ws) + xb;
    }
    if (any_shape)
        return generic(xin, w, s, scale_mode, bias, nullptr, nullptr, 0, nullptr, res, out, m, n,
                       k, scale_mode ? k : gs, 4, st);
    if (lb) {
        uint8_t *rec = static_cast<uint8_t *>(tail);
        float *part =
            reinterpret_cast<float *>(rec + up256(limb_records_bytes((int)m, (int)k)));
        if ((rc = limb_prep(xin, rec, (int)m, (int)k, st))) return rc;
        LimbParams q = limb_params(xin, rec, w, s, bias, out, m, n, k, gs, scale_mode);
        q.res = res;
        return w4_limb(q, part, st);
    }
    if (mf) {
        MfmaParams q = mfma_params(xin, w, s, bias, out, m, n, k, gs);
        q.res = res;
        q.v2 = v2 ? 1 : 0;
        q.scale_mode = scale_mode;
        return w4_mfma(q, epi, static_cast<float *>(tail), st);
    }
    W4Params p = w4_params(xin, w, s, bias, out, m, n, k, gs);
    p.res = res;
    p.v2 = v2 ? 1 : 0;
    p.scale_mode = scale_mode;
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
    TB_REQUIRE(k <= (1 << 30) && n < (1ll << 31) && m < (1ll << 31), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": dimension too large");
    TB_REQUIRE(aligned(x, 4) && aligned(s, 4), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": x and scales must be 4-byte aligned device pointers");
    return TB_OK;
}

// INT8 shapes the streaming GEMV takes: K a multiple of 32 within one pass's
// split-K range, 16-byte aligned x and w.  Others run the any-shape GEMV.
static bool w8_fast(const float *x, const void *w, int64_t k) {
    return k % 32 == 0 && k <= kMaxGemvK && aligned(x, 16) && aligned(w, 16);
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

// The any-shape GEMV over INT4 grouped (scale_mode 0), per-row (1) or scalar
// (2) scales, or INT8 (bits 8, scale_mode 1 / 2).
static int generic(const float *x, const void *w0, const float *s0, int mode0, const float *b0,
                   const void *w1, const float *s1, int mode1, const float *b1,
                   const float *res, float *y, int64_t m, int64_t n, int64_t k, int64_t gs,
                   int bits, hipStream_t st) {
    GenericParams g{};
    g.x = x; g.w0 = w0; g.s0 = s0; g.b0 = b0; g.w1 = w1; g.s1 = s1; g.b1 = b1;
    g.res = res; g.y = y; g.m = m; g.n = n; g.k = k; g.group = gs;
    g.scale_mode0 = mode0; g.scale_mode1 = mode1; g.bits = bits;
    return gemv_generic(g, st);
}

// ---- fused SwiGLU MLP (INT4), shared by the workspace and no-alloc entries ----
struct MlpW4 {
    const float *x;
    const uint8_t *gate_w;
    const float *gate_s, *gate_b;
    const uint8_t *up_w;
    const float *up_s, *up_b;
    const uint8_t *down_w;
    const float *down_s, *down_b, *residual;
    float *out;
    int64_t m, k, inter, n_out, gs;
};

static int mlp_w4_check(const MlpW4 &a, const char *op) {
    int rc = check_w4(a.x, a.gate_w, a.gate_s, a.m, a.inter, a.k, a.gs, op);
    if (rc) return rc;
    rc = check_w4(a.x, a.up_w, a.up_s, a.m, a.inter, a.k, a.gs, op);
    if (rc) return rc;
    TB_REQUIRE(a.down_w && a.down_s && a.out && a.inter > 0 && a.n_out >= 0, TB_ERR_UNSUPPORTED,
               std::string("TB_UNSUPPORTED: ") + op + ": null down weight or output");
    return TB_OK;
}

// 0: any-shape GEMVs; 1: FP32-MFMA pair; 2: GEMV passes; 3: small-batch f16 MFMA
static int mlp_w4_path(const MlpW4 &a) {
    if (limb_fast(a.x, a.gate_w, a.m, a.inter, a.k, a.gs, false, true) &&
        aligned(a.up_w, 16) &&
        limb_fast(a.x, a.down_w, a.m, a.n_out, a.inter, a.gs, false, false))
        return 3;
    if (!w4_fast(a.x, a.gate_w, a.m, a.k, a.gs, false) || !aligned(a.up_w, 16) ||
        !w4_fast(a.x, a.down_w, a.m, a.inter, a.gs, false))
        return 0;
    return a.m >= mfma_min_m() ? 1 : 2;
}

// Scratch: h [m, inter] f32, then the MFMA split-K partials (path 1), the
// chunk records of x and of h (path 2) or their f16-limb records (path 3).
// W4A8 semantics (tb_set_vnni_semantics) at group 64: the reference rounds x to
// bytes before the gate / up pair (fused_ops.rs:215-232) and h before the down
// projection, which is itself a group-64 GEMV (fused_ops.rs:409-421).
static bool mlp_a8(const MlpW4 &a) { return a.gs == 64 && vnni_semantics(); }

static size_t mlp_w4_scratch_main(const MlpW4 &a);

// [path scratch | x' (m x k) | h' (m x inter)], the last two under W4A8 only.
static size_t mlp_w4_scratch_bytes(const MlpW4 &a) {
    const size_t main = mlp_w4_scratch_main(a);
    if (!mlp_a8(a)) return main;
    return up256(main) + up256((size_t)a.m * (size_t)a.k * sizeof(float)) +
           up256((size_t)a.m * (size_t)a.inter * sizeof(float));
}

static size_t mlp_w4_scratch_main(const MlpW4 &a) {
    const size_t hb = up256((size_t)a.m * (size_t)a.inter * sizeof(float));
    switch (mlp_w4_path(a)) {
        case 0: return hb;
        case 3: {
            return hb + up256(limb_records_bytes((int)a.m, (int)a.k)) +
                   up256(limb_records_bytes((int)a.m, (int)a.inter)) +
                   std::max(limb_partials_bytes((int)a.m, (int)a.inter, (int)a.k, true),
                            limb_partials_bytes((int)a.m, (int)a.n_out, (int)a.inter, false));
        }
        case 1: {
            const size_t pg = w4_mfma_partials_bytes((int)a.m, (int)a.inter, (int)a.k, true);
            const size_t pd = w4_mfma_partials_bytes((int)a.m, (int)a.n_out, (int)a.inter, false);
            return hb + std::max(pg, pd);
        }
        default: return hb + up256(xq_bytes(a.m, a.k)) + xq_bytes(a.m, a.inter);
    }
}

// out = [residual +] down(silu(gate(x)) * up(x)) with `ws` of at least
// mlp_w4_scratch_bytes(a) bytes (fused_swiglu_mlp_w4a32, fused_ops.rs:138-424).
static int mlp_w4_run(const MlpW4 &a, void *ws, hipStream_t st) {
    int rc;
    const int64_t m = a.m, k = a.k, inter = a.inter, n_out = a.n_out, gs = a.gs;
    float *h = static_cast<float *>(ws);
    const size_t hb = up256((size_t)m * (size_t)inter * sizeof(float));
    const int path = mlp_w4_path(a);
    // W4A8: x -> x' here, h -> h' before the down projection (the byte rounding
    // of each activation row, written back as q * s_x).
    const bool a8 = mlp_a8(a);
    float *xa = nullptr, *ha = nullptr;
    const float *x = a.x;
    if (a8) {
        xa = reinterpret_cast<float *>(static_cast<char *>(ws) + up256(mlp_w4_scratch_main(a)));
        ha = reinterpret_cast<float *>(reinterpret_cast<char *>(xa) +
                                       up256((size_t)m * (size_t)k * sizeof(float)));
        if ((rc = act_u8(a.x, xa, m, k, st))) return rc;
        x = xa;
    }
    const float *hin = a8 ? ha : h;   // the down projection's input
    if (path == 0) {
        // Shapes outside the streaming kernels: h by the any-shape GEMV, then the
        // down projection by whichever path its own shape takes.
        rc = generic(x, a.gate_w, a.gate_s, 0, a.gate_b, a.up_w, a.up_s, 0, a.up_b, nullptr, h, m,
                     inter, k, gs, 4, st);
        if (rc) return rc;
        if (a8 && (rc = act_u8(h, ha, m, inter, st))) return rc;
        return generic(hin, a.down_w, a.down_s, 0, a.down_b, nullptr, nullptr, 0, nullptr,
                       a.residual, a.out, m, n_out, inter, gs, 4, st);
    }
    if (path == 3) {
        // prep(x) -> gate/up + SwiGLU, which also writes h's records -> down
        // (W4A8: h' and its records replace them)
        uint8_t *xr = static_cast<uint8_t *>(ws) + hb;
        uint8_t *hr = xr + up256(limb_records_bytes((int)m, (int)k));
        float *part =
            reinterpret_cast<float *>(hr + up256(limb_records_bytes((int)m, (int)inter)));
        if ((rc = limb_prep(x, xr, (int)m, (int)k, st))) return rc;
        LimbParams g = limb_params(x, xr, a.gate_w, a.gate_s, a.gate_b, h, m, inter, k, gs);
        g.w1 = a.up_w; g.s1 = a.up_s; g.b1 = a.up_b;
        g.rec_out = hr;
        if ((rc = w4_limb(g, part, st))) return rc;
        if (a8 && ((rc = act_u8(h, ha, m, inter, st)) ||
                   (rc = limb_prep(ha, hr, (int)m, (int)inter, st))))
            return rc;
        LimbParams d = limb_params(hin, hr, a.down_w, a.down_s, a.down_b, a.out, m, n_out, inter,
                                   gs);
        d.res = a.residual;
        return w4_limb(d, part, st);
    }
    if (path == 1) {
        float *part = reinterpret_cast<float *>(static_cast<char *>(ws) + hb);
        MfmaParams g = mfma_params(x, a.gate_w, a.gate_s, a.gate_b, h, m, inter, k, gs);
        g.w1 = a.up_w; g.s1 = a.up_s; g.b1 = a.up_b;
        if ((rc = w4_mfma(g, EPI_SWIGLU, part, st))) return rc;
        if (a8 && (rc = act_u8(h, ha, m, inter, st))) return rc;
        MfmaParams d = mfma_params(hin, a.down_w, a.down_s, a.down_b, a.out, m, n_out, inter, gs);
        d.res = a.residual;
        return w4_mfma(d, a.residual ? EPI_RESID : EPI_PLAIN, part, st);
    }
    uint32_t *xq = reinterpret_cast<uint32_t *>(static_cast<char *>(ws) + hb);
    uint32_t *hq = reinterpret_cast<uint32_t *>(static_cast<char *>(ws) + hb +
                                                up256(xq_bytes(m, k)));
    W4Params p = w4_params(x, a.gate_w, a.gate_s, a.gate_b, h, m, inter, k, gs);
    p.w1 = a.up_w; p.s1 = a.up_s; p.b1 = a.up_b;
    W4Params d = w4_params(hin, a.down_w, a.down_s, a.down_b, a.out, m, n_out, inter, gs);
    d.res = a.residual;
    const int depi = a.residual ? EPI_RESID : EPI_PLAIN;
    if (m == 1) {
        // One row: the gate/up epilogue writes h's chunk records as well, so the
        // down projection needs no separate record pass (W4A8: h' and its
        // records in one pass instead).
        if ((rc = xquant(x, xq, 1, (int)k, st))) return rc;
        p.xq = xq;
        p.rec_out = a8 ? nullptr : hq;
        if ((rc = w4_gemv(p, EPI_SWIGLU, st))) return rc;
        if (a8 && (rc = act_rec(h, ha, hq, 1, inter, st))) return rc;
        d.xq = hq;
        return w4_gemv(d, depi, st);
    }
    if ((rc = w4_rows(p, EPI_SWIGLU, m, xq, true, st))) return rc;
    if (a8 && (rc = act_u8(h, ha, m, inter, st))) return rc;
    return w4_rows(d, depi, m, hq, true, st);
}

// ---- the no-allocation MLP entry point ----
// Scratch of tb_fused_swiglu_mlp_w4a32_noalloc, in the code object's static
// device memory: every GPU the library runs on holds one copy of
// kNoAllocScratchBytes until the process ends.  `scratch` names the host-side
// stand-in of the array; its device address (per device) comes from
// hipGetSymbolAddress and is the only form passed to kernels.
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];   // device address of `scratch` per device, or null
}  // namespace

// The current device's address of `scratch`, looked up on the first call per
// device with that device current (no allocation).
static int noalloc_scratch(void **out) {
    int dev = 0;
    TB_HIP(hipGetDevice(&dev));
    TB_REQUIRE(dev >= 0 && dev < kMaxDevices, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: no-alloc entry points support device ids below " +
                   std::to_string(kMaxDevices));
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        TB_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
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
    TB_REQUIRE(group_size >= 1, TB_ERR_VALUE,
               "quantize_weight_int4_grouped: group_size must be positive, got " +
                   std::to_string(group_size));
    TB_REQUIRE(n >= 0 && k > 0 && k <= (1 << 30), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: quantize_weight_int4_grouped: bad shape");
    TB_REQUIRE(k % group_size == 0, TB_ERR_VALUE,
               "Weight dimension K=" + std::to_string(k) + " must be divisible by group_size=" +
                   std::to_string(group_size) + ". Consider padding the weight tensor along dim 1 "
                   "to a multiple of " + std::to_string(group_size) + ".");
    // two nibbles per byte: the reference's (low | high) has no partner for
    // the last element of an odd K (its shapes differ and torch raises)
    TB_REQUIRE(k % 2 == 0, TB_ERR_VALUE,
               "quantize_weight_int4_grouped: K=" + std::to_string(k) +
                   " is odd: the nibble pairs (K + 1) / 2 low and (K - 1) / 2 high differ");
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
    SampleParams prm{};
    prm.temperature = temperature;
    prm.top_p = top_p;
    prm.penalty = repetition_penalty;
    prm.k = (int)k;
    prm.greedy = greedy ? 1 : 0;
    prm.seed = seed;
    prm.counter = counter;
    const size_t cand = (size_t)sample_scratch_items(vocab);
    const size_t bytes = up256(sizeof(SampleParams)) + up256(sizeof(SampleOut)) +
                         3 * up256(cand * 4) + up256(kSampleLists * 4);
    WsLease lease;
    int rc = workspace(bytes, (hipStream_t)stream, lease);
    if (rc) return rc;
    void *ws = lease.ptr;
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
    sc.p = reinterpret_cast<float *>(w);
    w += up256(cand * 4);
    sc.cnt = reinterpret_cast<int *>(w);
    hipStream_t st = (hipStream_t)stream;
    TB_HIP(hipMemcpyAsync(dprm, &prm, sizeof(prm), hipMemcpyHostToDevice, st));
    rc = launch_sample(logits, (int)vocab, recent, (int)n_recent, dprm, sc, dout, st,
                       k > kSampleMaxK);
    if (rc) return rc;
    SampleOut ho{};
    TB_HIP(hipMemcpyAsync(&ho, dout, sizeof(ho), hipMemcpyDeviceToHost, st));
    TB_HIP(hipStreamSynchronize(st));
    *token_out = ho.token;
    if (u_out) *u_out = ho.u;
    return TB_OK;
}

int tb_release_stream_workspace(void *stream) {
    int dev = 0;
    TB_HIP(hipGetDevice(&dev));
    std::unique_ptr<StreamScratch> sc;
    {
        std::lock_guard<std::mutex> lk(g_ws_mu);
        auto it = g_ws.find({dev, reinterpret_cast<uintptr_t>(stream)});
        if (it == g_ws.end()) return TB_OK;
        sc = std::move(it->second);
        g_ws.erase(it);
    }
    {
        // an op still enqueueing on this stream finishes first
        std::lock_guard<std::mutex> lk(sc->mu);
    }
    // Work already enqueued on the stream may still read the buffers.
    TB_HIP(hipDeviceSynchronize());
    for (void *p : sc->retired) TB_HIP(hipFree(p));
    if (sc->ptr) TB_HIP(hipFree(sc->ptr));
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
    if (limb_fast(x, gate_w, m, inter, k, group_size, false, true) && aligned(up_w, 16)) {
        WsLease lease;
        const size_t rb = up256(limb_records_bytes((int)m, (int)k));
        if ((rc = workspace(rb + limb_partials_bytes((int)m, (int)inter, (int)k, true),
                            (hipStream_t)stream, lease)))
            return rc;
        uint8_t *rec = static_cast<uint8_t *>(lease.ptr);
        if ((rc = limb_prep(x, rec, (int)m, (int)k, (hipStream_t)stream))) return rc;
        LimbParams q = limb_params(x, rec, gate_w, gate_s, gate_b, h, m, inter, k, group_size);
        q.w1 = up_w; q.s1 = up_s; q.b1 = up_b;
        return w4_limb(q, reinterpret_cast<float *>(rec + rb), (hipStream_t)stream);
    }
    if (!w4_fast(x, gate_w, m, k, group_size, false) || !aligned(up_w, 16))
        return generic(x, gate_w, gate_s, 0, gate_b, up_w, up_s, 0, up_b, nullptr, h, m, inter, k,
                       group_size, 4, (hipStream_t)stream);
    if (m >= mfma_min_m()) {
        MfmaParams q = mfma_params(x, gate_w, gate_s, gate_b, h, m, inter, k, group_size);
        q.w1 = up_w; q.s1 = up_s; q.b1 = up_b;
        return mfma_ws(q, EPI_SWIGLU, (hipStream_t)stream);
    }
    WsLease lease;
    rc = workspace(xq_bytes(m, k), (hipStream_t)stream, lease);
    if (rc) return rc;
    void *ws = lease.ptr;
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
    const MlpW4 a{x, gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s, down_b,
                  residual, out, m, k, inter, n_out, group_size};
    int rc = mlp_w4_check(a, "fused_swiglu_mlp_w4a32");
    if (rc || m == 0 || n_out == 0) return rc;
    hipStream_t st = (hipStream_t)stream;
    WsLease lease;
    if ((rc = workspace(mlp_w4_scratch_bytes(a), st, lease))) return rc;
    return mlp_w4_run(a, lease.ptr, st);
}

int tb_fused_swiglu_mlp_w4a32_noalloc(const float *x, const uint8_t *gate_w,
                                      const float *gate_s, const float *gate_b,
                                      const uint8_t *up_w, const float *up_s, const float *up_b,
                                      const uint8_t *down_w, const float *down_s,
                                      const float *down_b, const float *residual, float *out,
                                      int64_t m, int64_t k, int64_t inter, int64_t n_out,
                                      int64_t group_size, void *stream) {
    const MlpW4 a{x, gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s, down_b,
                  residual, out, m, k, inter, n_out, group_size};
    int rc = mlp_w4_check(a, "fused_swiglu_mlp_w4a32_noalloc");
    if (rc || m == 0 || n_out == 0) return rc;
    const size_t need = mlp_w4_scratch_bytes(a);
    TB_REQUIRE(need <= kNoAllocScratchBytes, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: fused_swiglu_mlp_w4a32_noalloc: this shape needs " +
                   std::to_string(need) + " bytes of scratch; the static scratch holds " +
                   std::to_string(kNoAllocScratchBytes) +
                   " (use tb_fused_swiglu_mlp_w4a32, which allocates)");
    void *ws = nullptr;
    if ((rc = noalloc_scratch(&ws))) return rc;
    return mlp_w4_run(a, ws, (hipStream_t)stream);
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
    TB_REQUIRE(w4_fast(x, w_packed, m, k, group_size, false), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: w4a32_gemv_xq: records need K % 32 == 0, a power-of-two group "
               ">= 32 and K <= " + std::to_string(kMaxGemvK));
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
    TB_REQUIRE(w4_fast(x, gate_w, m, k, group_size, false) && aligned(up_w, 16),
               TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: swiglu_w4a32_xq: records need K % 32 == 0, a power-of-two group "
               ">= 32 and K <= " + std::to_string(kMaxGemvK));
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

int tb_w4a32_linear(const float *x, const uint8_t *w_packed, const float *scales, int64_t s_len,
                    const float *bias, float *out, int64_t m, int64_t n, int64_t k, void *stream) {
    int rc = check_w4(x, w_packed, scales, m, n, k, 2, "w4a32_linear");
    if (rc) return rc;
    TB_REQUIRE(out, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: w4a32_linear: null output");
    TB_REQUIRE(s_len == 1 || s_len == n, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: w4a32_linear: scales must have 1 or N elements");
    if (m == 0 || n == 0) return TB_OK;
    // y = dot * s + b with one scale per row or one scalar (gemv.rs:1114-1180)
    return linear_w4(x, w_packed, scales, false, bias, nullptr, out, m, n, k, 32,
                     (hipStream_t)stream, s_len > 1 ? 1 : 2);
}

int tb_quantize_weight_int4(const float *w, uint8_t *packed, float *scales, int64_t n, int64_t k,
                            void *stream) {
    TB_REQUIRE(w && packed && scales, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: quantize_weight_int4: null pointer");
    TB_REQUIRE(n >= 0 && k > 0 && k <= (1 << 30) && n < (1ll << 31), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: quantize_weight_int4: bad shape");
    TB_REQUIRE(aligned(w, 4) && aligned(scales, 4), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: quantize_weight_int4: misaligned device pointer");
    return quantize_int4_rows(w, packed, scales, n, k, (hipStream_t)stream);
}

int tb_w8a32_linear(const float *x, const int8_t *w, const float *scales, int64_t s_len,
                    const float *bias, float *out, int64_t m, int64_t n, int64_t k,
                    void *stream) {
    int rc = check_w8(x, w, scales, s_len, m, n, k, "w8a32_linear");
    if (rc) return rc;
    TB_REQUIRE(out, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: w8a32_linear: null output");
    if (m == 0 || n == 0) return TB_OK;
    if (!w8_fast(x, w, k))
        return generic(x, w, scales, s_len > 1 ? 1 : 2, bias, nullptr, nullptr, 0, nullptr,
                       nullptr, out, m, n, k, 1, 8, (hipStream_t)stream);
    DenseParams p{};
    p.x = x; p.w0 = w; p.rs0 = scales; p.rs0_len = (int)s_len; p.b0 = bias; p.y = out;
    p.m = (int)m; p.n = (int)n; p.k = (int)k;
    return dense_rows(p, W_I8, EPI_PLAIN, m, (hipStream_t)stream);
}

int tb_fused_swiglu_mlp_w8a32(const float *x, const int8_t *gate_w, const float *gate_s,
                              int64_t gate_s_len, const float *gate_b, const int8_t *up_w,
                              const float *up_s, int64_t up_s_len, const float *up_b,
                              const int8_t *down_w, const float *down_s, int64_t down_s_len,
                              const float *down_b, const float *residual, float *out, int64_t m,
                              int64_t k, int64_t inter, int64_t n_out, void *stream) {
    // Each projection's scales are per row (N elements) or one per-tensor
    // scalar (fused_ops.rs:80-97 and gemv_w8a32's s_len).
    int rc = check_w8(x, gate_w, gate_s, gate_s_len, m, inter, k, "fused_swiglu_mlp_w8a32 gate");
    if (rc) return rc;
    rc = check_w8(x, up_w, up_s, up_s_len, m, inter, k, "fused_swiglu_mlp_w8a32 up");
    if (rc) return rc;
    TB_REQUIRE(out && (inter > 0 || n_out == 0), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: fused_swiglu_mlp_w8a32: null output");
    if (m == 0 || n_out == 0) return TB_OK;
    // down reads h [m, inter] from the workspace (x stands in for its checks)
    rc = check_w8(x, down_w, down_s, down_s_len, m, n_out, inter, "fused_swiglu_mlp_w8a32 down");
    if (rc) return rc;
    WsLease lease;
    rc = workspace((size_t)m * (size_t)inter * sizeof(float), (hipStream_t)stream, lease);
    if (rc) return rc;
    void *ws = lease.ptr;
    float *h = static_cast<float *>(ws);
    hipStream_t st = (hipStream_t)stream;
    if (!w8_fast(x, gate_w, k) || !aligned(up_w, 16) || !w8_fast(h, down_w, inter)) {
        rc = generic(x, gate_w, gate_s, gate_s_len > 1 ? 1 : 2, gate_b, up_w, up_s,
                     up_s_len > 1 ? 1 : 2, up_b, nullptr, h, m, inter, k, 1, 8, st);
        if (rc) return rc;
        return generic(h, down_w, down_s, down_s_len > 1 ? 1 : 2, down_b, nullptr, nullptr, 0,
                       nullptr, residual, out, m, n_out, inter, 1, 8, st);
    }
    DenseParams p{};
    p.x = x; p.w0 = gate_w; p.rs0 = gate_s; p.rs0_len = (int)gate_s_len; p.b0 = gate_b;
    p.w1 = up_w; p.rs1 = up_s; p.rs1_len = (int)up_s_len; p.b1 = up_b;
    p.y = h; p.m = (int)m; p.n = (int)inter; p.k = (int)k;
    rc = dense_rows(p, W_I8, EPI_SWIGLU, m, st);
    if (rc) return rc;
    DenseParams d{};
    d.x = h; d.w0 = down_w; d.rs0 = down_s; d.rs0_len = (int)down_s_len; d.b0 = down_b;
    d.res = residual; d.y = out; d.m = (int)m; d.n = (int)n_out; d.k = (int)inter;
    return dense_rows(d, W_I8, residual ? EPI_RESID : EPI_PLAIN, m, st);
}

}  // extern "C"

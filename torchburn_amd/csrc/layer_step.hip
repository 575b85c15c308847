// Per-layer decode steps on caller-owned weights, KV caches and the RoPE row
// of the current position (declared in include/tbhip.h):
//   tb_fused_attention_step_w4a32 / _w8a32  <- fused_attention_step_w4a32 /
//       _w8a32 (reference src/quantization/fused_ops.rs:891-1062, 718-888);
//   tb_fused_transformer_layer_step_w4a32   <- fused_transformer_layer_step_w4a32
//       (src/quantization/fused_transformer.rs:16-376).
// They run the decoder's kernels one layer at a time: the QKV projection with
// bias, RoPE and the KV-cache append in its epilogue, split-KV attention with
// its merge, the O projection (and, for the layer step, RMSNorm, the residual
// adds and the SwiGLU MLP).  The current position lives in a device-side
// DecState, set by a one-thread kernel so the sequence can be captured.
#include <string>

#include <limits.h>

#include <algorithm>

#include "decode.hpp"
#include "gemv_dense.hpp"
#include "tb_common.hpp"
#include "v2_layout.hpp"
#include "w4_gemv.hpp"

namespace tb {

namespace {

bool is_aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

__global__ void k_set_pos(DecState *st, int pos) {
    st->token = 0;
    st->pos = pos;
    st->step = 0;
    st->argmax = 0;
}

size_t up256(size_t b) { return (b + 255) & ~(size_t)255; }
size_t recs(int64_t k) { return (size_t)(k / 32) * kXRecDwords * sizeof(uint32_t); }

// Device scratch of one layer step, carved from the library workspace.
struct LayerWs {
    DecState *state;
    float *qkv;       // [hq*hd + 2*hkv*hd]: q after RoPE (k, v go to the caches)
    float *part;      // attention split partials
    float *attn;      // [hq*hd]
    uint32_t *xq_a;   // records of attn (INT4)
    float *xn;        // [H] normed x
    uint32_t *xq_h;   // records of xn (INT4)
    float *h;         // [I] SwiGLU output
    uint32_t *xq_i;   // records of h (INT4)
    float *xa;        // W4A8: x' = q * s_x of the current projection input
};

int layer_ws(int64_t H, int64_t I, int hq, int hkv, int hd, int max_seq, LayerWs &w,
             WsLease &lease, hipStream_t st) {
    const size_t qkv_n = (size_t)(hq + 2 * hkv) * hd;
    const size_t part_n = (size_t)hq * attn_nsplit(max_seq) * (hd + 4);
    size_t off[10], o = 0;
    const size_t xa_n = (size_t)std::max<int64_t>({H, (int64_t)hq * hd, I});
    const size_t sz[10] = {up256(sizeof(DecState)), up256(qkv_n * 4), up256(part_n * 4),
                           up256((size_t)hq * hd * 4), up256(recs((int64_t)hq * hd)),
                           up256((size_t)H * 4), up256(recs(H)), up256((size_t)I * 4),
                           up256(recs(I)), up256(xa_n * 4)};
    for (int i = 0; i < 10; ++i) {
        off[i] = o;
        o += sz[i];
    }
    int rc = workspace(o, st, lease);
    if (rc) return rc;
    char *b = static_cast<char *>(lease.ptr);
    w.state = reinterpret_cast<DecState *>(b + off[0]);
    w.qkv = reinterpret_cast<float *>(b + off[1]);
    w.part = reinterpret_cast<float *>(b + off[2]);
    w.attn = reinterpret_cast<float *>(b + off[3]);
    w.xq_a = reinterpret_cast<uint32_t *>(b + off[4]);
    w.xn = reinterpret_cast<float *>(b + off[5]);
    w.xq_h = reinterpret_cast<uint32_t *>(b + off[6]);
    w.h = reinterpret_cast<float *>(b + off[7]);
    w.xq_i = reinterpret_cast<uint32_t *>(b + off[8]);
    w.xa = reinterpret_cast<float *>(b + off[9]);
    return TB_OK;
}

// W4A8 semantics (tb_set_vnni_semantics) at group 64: on an AVX-512 VNNI host
// every group-64 projection of the reference's layer steps rounds its input
// to bytes (gemv.rs:1559-1563 under fused_ops.rs:932-1049 and
// fused_transformer.rs:102-241; the SwiGLU pair fused_transformer.rs:299).
bool a8_on(int bits, int64_t gs) { return bits == 4 && gs == 64 && vnni_semantics(); }

// Shape checks shared by the three entry points (the reference indexes its
// slices with these sizes; it panics where this returns TB_UNSUPPORTED).
int check_attn(const char *what, int64_t H, int64_t offset, int64_t max_seq, int64_t hq,
               int64_t hkv, int64_t hd, const float *k_cache, const float *v_cache,
               const float *cos, const float *sin) {
    const std::string op(what);
    TB_REQUIRE(k_cache && v_cache && cos && sin, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": null cache or RoPE row");
    TB_REQUIRE(hq > 0 && hkv > 0 && hq % hkv == 0 && hq / hkv <= 64, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": num_heads must be a multiple of num_kv_heads");
    TB_REQUIRE(hd == 64 || hd == 128, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": head_dim must be 64 or 128");
    TB_REQUIRE(H > 0 && H % 32 == 0 && H <= kMaxHidden, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": hidden size must be a multiple of 32 and <= " +
                   std::to_string(kMaxHidden));
    TB_REQUIRE(max_seq > 0 && max_seq <= (int64_t)kMaxTiles * kAttnTile, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": cache length out of range");
    TB_REQUIRE(offset >= 0 && offset < max_seq, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": offset " + std::to_string(offset) +
                   " outside the cache of length " + std::to_string(max_seq));
    TB_REQUIRE(is_aligned(k_cache, 16) && is_aligned(v_cache, 16), TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": caches must be 16-byte aligned device pointers");
    return TB_OK;
}

int gshift_from(int64_t gs) { return gs == 32 ? 5 : (gs == 64 ? 6 : -1); }

// One projection of the layer: INT4 (records xq of x) or INT8 per-channel.
struct Proj {
    int bits;
    const void *w;
    const float *s;
    int64_t s_len;   // INT8 scales: 1 or n
    const float *b;
};

int project(const Proj &P, const float *x, const uint32_t *xq, const Proj *P2, const float *res,
            float *y, int64_t n, int64_t k, int gshift, int epi, const RopeArgs *rope,
            hipStream_t st) {
    if (P.bits == 4) {
        W4Params p{};
        p.x = x; p.xq = xq;
        p.w0 = static_cast<const uint8_t *>(P.w); p.s0 = P.s; p.b0 = P.b;
        if (P2) { p.w1 = static_cast<const uint8_t *>(P2->w); p.s1 = P2->s; p.b1 = P2->b; }
        p.res = res; p.y = y; p.m = 1; p.n = (int)n; p.k = (int)k; p.gshift = gshift;
        if (rope) p.rope = *rope;
        return w4_gemv(p, epi, st);
    }
    DenseParams p{};
    p.x = x; p.w0 = P.w; p.rs0 = P.s; p.rs0_len = (int)P.s_len; p.b0 = P.b;
    if (P2) { p.w1 = P2->w; p.rs1 = P2->s; p.rs1_len = (int)P2->s_len; p.b1 = P2->b; }
    p.res = res; p.y = y; p.m = 1; p.n = (int)n; p.k = (int)k;
    if (rope) p.rope = *rope;
    return dense_gemv(p, W_I8, epi, st);
}

// QKV (+bias, RoPE, KV append) -> attention -> O (+bias, + residual when res).
// xq: records of x (INT4); out may alias res (in-place residual).  a8: the
// attention output is byte-rounded (x' and its records) before O.
int attention_block(const Proj &qkv, const Proj &o, const float *x, const uint32_t *xq,
                    float *kc, float *vc, const float *cos, const float *sin, const float *res,
                    float *out, int64_t H, int hq, int hkv, int hd, int max_seq, int gshift,
                    bool a8, const LayerWs &w, hipStream_t st) {
    // cos / sin hold one position's row: a table stride of 0 makes every
    // position read it.
    RopeArgs ra{&w.state->pos, cos, sin, kc, vc, hq, hkv, hd, max_seq, 0};
    const int64_t nq = (int64_t)(hq + 2 * hkv) * hd;
    int rc = project(qkv, x, xq, nullptr, nullptr, w.qkv, nq, H, gshift, EPI_ROPE, &ra, st);
    if (rc) return rc;
    const bool q4 = o.bits == 4;
    // The per-layer path scores every position (no cap: fused_ops.rs:997-1040).
    rc = launch_attention(w.state, w.qkv, kc, vc, w.part, w.attn, q4 && !a8 ? w.xq_a : nullptr,
                          hq, hkv, hd, max_seq, INT_MAX, st);
    if (rc) return rc;
    const float *ain = w.attn;
    if (a8) {
        if ((rc = act_rec(w.attn, w.xa, w.xq_a, 1, (int64_t)hq * hd, st))) return rc;
        ain = w.xa;
    }
    return project(o, ain, w.xq_a, nullptr, res, out, H, (int64_t)hq * hd, gshift,
                   res ? EPI_RESID : EPI_PLAIN, nullptr, st);
}

int set_pos(const LayerWs &w, int64_t offset, hipStream_t st) {
    hipLaunchKernelGGL(k_set_pos, dim3(1), dim3(1), 0, st, w.state, (int)offset);
    TB_LAUNCHED();
    return TB_OK;
}

int attention_step(const char *what, int bits, const float *x, const void *qkv_w,
                   const float *qkv_s, int64_t qkv_s_len, const float *qkv_b, const void *o_w,
                   const float *o_s, int64_t o_s_len, const float *o_b, float *k_cache,
                   float *v_cache, const float *cos, const float *sin, float *out, int64_t H,
                   int64_t offset, int64_t max_seq, int64_t hq, int64_t hkv, int64_t hd,
                   int64_t group_size, hipStream_t st) {
    const std::string op(what);
    TB_REQUIRE(x && qkv_w && qkv_s && o_w && o_s && out, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": null pointer");
    int rc = check_attn(what, H, offset, max_seq, hq, hkv, hd, k_cache, v_cache, cos, sin);
    if (rc) return rc;
    const int gshift = bits == 4 ? gshift_from(group_size) : 5;
    TB_REQUIRE(gshift > 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": group_size must be 32 or 64");
    if (bits == 4)
        TB_REQUIRE(H % group_size == 0 && (hq * hd) % group_size == 0, TB_ERR_UNSUPPORTED,
                   "TB_UNSUPPORTED: " + op + ": K must be a multiple of group_size");
    const int64_t nq = (hq + 2 * hkv) * hd;
    if (bits == 8)
        TB_REQUIRE((qkv_s_len == 1 || qkv_s_len == nq) && (o_s_len == 1 || o_s_len == H),
                   TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: " + op + ": scales must have 1 or N elements");
    TB_REQUIRE(is_aligned(x, 16) && is_aligned(qkv_w, 16) && is_aligned(o_w, 16) &&
                   is_aligned(out, 16),
               TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: " + op + ": 16-byte aligned device pointers required");
    LayerWs w;
    WsLease lease;
    if ((rc = layer_ws(H, 0, (int)hq, (int)hkv, (int)hd, (int)max_seq, w, lease, st))) return rc;
    if ((rc = set_pos(w, offset, st))) return rc;
    const bool a8 = a8_on(bits, group_size);
    const float *xin = x;
    if (a8) {
        if ((rc = act_rec(x, w.xa, w.xq_h, 1, H, st))) return rc;
        xin = w.xa;
    } else if (bits == 4 && (rc = xquant(x, w.xq_h, 1, (int)H, st))) {
        return rc;
    }
    const Proj qkv{bits, qkv_w, qkv_s, qkv_s_len, qkv_b};
    const Proj o{bits, o_w, o_s, o_s_len, o_b};
    return attention_block(qkv, o, xin, w.xq_h, k_cache, v_cache, cos, sin, nullptr, out, H,
                           (int)hq, (int)hkv, (int)hd, (int)max_seq, gshift, a8, w, st);
}

}  // namespace

}  // namespace tb

using namespace tb;

extern "C" {

int tb_fused_attention_step_w4a32(const float *x, const uint8_t *qkv_w, const float *qkv_s,
                                  const float *qkv_b, const uint8_t *o_w, const float *o_s,
                                  const float *o_b, float *k_cache, float *v_cache,
                                  const float *cos, const float *sin, float *out, int64_t hidden,
                                  int64_t offset, int64_t max_seq, int64_t num_heads,
                                  int64_t num_kv_heads, int64_t head_dim, int64_t group_size,
                                  void *stream) {
    return attention_step("fused_attention_step_w4a32", 4, x, qkv_w, qkv_s, 0, qkv_b, o_w, o_s, 0,
                          o_b, k_cache, v_cache, cos, sin, out, hidden, offset, max_seq,
                          num_heads, num_kv_heads, head_dim, group_size, (hipStream_t)stream);
}

int tb_fused_attention_step_w8a32(const float *x, const int8_t *qkv_w, const float *qkv_s,
                                  int64_t qkv_s_len, const float *qkv_b, const int8_t *o_w,
                                  const float *o_s, int64_t o_s_len, const float *o_b,
                                  float *k_cache, float *v_cache, const float *cos,
                                  const float *sin, float *out, int64_t hidden, int64_t offset,
                                  int64_t max_seq, int64_t num_heads, int64_t num_kv_heads,
                                  int64_t head_dim, void *stream) {
    return attention_step("fused_attention_step_w8a32", 8, x, qkv_w, qkv_s, qkv_s_len, qkv_b, o_w,
                          o_s, o_s_len, o_b, k_cache, v_cache, cos, sin, out, hidden, offset,
                          max_seq, num_heads, num_kv_heads, head_dim, 32, (hipStream_t)stream);
}

int tb_fused_transformer_layer_step_w4a32(
    float *x, const float *input_norm_w, const uint8_t *qkv_w, const float *qkv_s,
    const float *qkv_b, const uint8_t *o_w, const float *o_s, const float *o_b,
    const float *post_norm_w, const uint8_t *gate_w, const float *gate_s, const float *gate_b,
    const uint8_t *up_w, const float *up_s, const float *up_b, const uint8_t *down_w,
    const float *down_s, const float *down_b, float *k_cache, float *v_cache, const float *cos,
    const float *sin, int64_t hidden, int64_t intermediate, int64_t offset, int64_t max_seq,
    int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t group_size, double eps,
    void *stream) {
    const char *what = "fused_transformer_layer_step_w4a32";
    const std::string op(what);
    hipStream_t st = (hipStream_t)stream;
    TB_REQUIRE(x && input_norm_w && qkv_w && qkv_s && o_w && o_s && post_norm_w && gate_w &&
                   gate_s && up_w && up_s && down_w && down_s,
               TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: " + op + ": null pointer");
    int rc = check_attn(what, hidden, offset, max_seq, num_heads, num_kv_heads, head_dim,
                        k_cache, v_cache, cos, sin);
    if (rc) return rc;
    const int gshift = gshift_from(group_size);
    TB_REQUIRE(gshift > 0, TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": group_size must be 32 or 64");
    TB_REQUIRE(intermediate > 0 && intermediate % 32 == 0 && intermediate % group_size == 0 &&
                   hidden % group_size == 0 && (num_heads * head_dim) % group_size == 0,
               TB_ERR_UNSUPPORTED,
               "TB_UNSUPPORTED: " + op + ": K dimensions must be multiples of group_size");
    TB_REQUIRE(is_aligned(x, 16) && is_aligned(input_norm_w, 16) && is_aligned(post_norm_w, 16) &&
                   is_aligned(qkv_w, 16) && is_aligned(o_w, 16) && is_aligned(gate_w, 16) &&
                   is_aligned(up_w, 16) && is_aligned(down_w, 16),
               TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: " + op + ": 16-byte aligned device pointers required");
    LayerWs w;
    WsLease lease;
    if ((rc = layer_ws(hidden, intermediate, (int)num_heads, (int)num_kv_heads, (int)head_dim,
                       (int)max_seq, w, lease, st)))
        return rc;
    if ((rc = set_pos(w, offset, st))) return rc;
    const float e = (float)eps;
    const int H = (int)hidden, I = (int)intermediate;
    const bool a8 = a8_on(4, group_size);
    // The input of a projection: xn with its records, or under W4A8 x' and its records.
    auto input = [&](const float *v, uint32_t *xq, int64_t k, const float **in) -> int {
        *in = v;
        if (!a8) return TB_OK;
        *in = w.xa;
        return act_rec(v, w.xa, xq, 1, k, st);
    };
    const float *in = nullptr;
    // 1. xn = RMSNorm(x) (+ its records), 2-6. attention block, x += O(attn)
    if ((rc = launch_rmsnorm(w.state, nullptr, x, input_norm_w, w.xn, a8 ? nullptr : w.xq_h, H, e,
                             st)) ||
        (rc = input(w.xn, w.xq_h, H, &in)))
        return rc;
    const Proj qkv{4, qkv_w, qkv_s, 0, qkv_b}, o{4, o_w, o_s, 0, o_b};
    rc = attention_block(qkv, o, in, w.xq_h, k_cache, v_cache, cos, sin, x, x, hidden,
                         (int)num_heads, (int)num_kv_heads, (int)head_dim, (int)max_seq, gshift,
                         a8, w, st);
    if (rc) return rc;
    // 8. xn = RMSNorm(x), 9. h = silu(gate xn + gb) * (up xn + ub), x += down h + db
    if ((rc = launch_rmsnorm(w.state, nullptr, x, post_norm_w, w.xn, a8 ? nullptr : w.xq_h, H, e,
                             st)) ||
        (rc = input(w.xn, w.xq_h, H, &in)))
        return rc;
    const Proj gate{4, gate_w, gate_s, 0, gate_b}, up{4, up_w, up_s, 0, up_b};
    rc = project(gate, in, w.xq_h, &up, nullptr, w.h, intermediate, hidden, gshift, EPI_SWIGLU,
                 nullptr, st);
    if (rc) return rc;
    if (a8) {
        if ((rc = input(w.h, w.xq_i, I, &in))) return rc;
    } else {
        if ((rc = xquant(w.h, w.xq_i, 1, I, st))) return rc;
        in = w.h;
    }
    const Proj down{4, down_w, down_s, 0, down_b};
    return project(down, in, w.xq_i, nullptr, x, x, hidden, intermediate, gshift, EPI_RESID,
                   nullptr, st);
}

}  // extern "C"

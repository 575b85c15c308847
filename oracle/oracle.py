"""ctypes binding for the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker (or the timed
CPU baseline) -- never as the thing measured or shipped.  The product path in
torchburn_amd/ never imports it.

Every function mirrors one C function in tb_oracle.c, which cites the
reference file:line it restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# TB_ORACLE_SO: another build of the same source, e.g. the sanitizer build of
# sanitize.sh; by default the Makefile's liboracle.so beside this file
_SO = os.environ.get("TB_ORACLE_SO") or os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i64 = C.c_int64
_vp = C.c_void_p


def build() -> None:
    """Compile liboracle.so with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = C.CDLL(_SO)
        L.orc_pack_int4.argtypes = [_i8p, _u8p, _i64, _i64]
        L.orc_unpack_int4.argtypes = [_u8p, _i8p, _i64, _i64]
        L.orc_quantize_int4_grouped.argtypes = [_f32p, _u8p, _f32p, _i64, _i64, _i64]
        L.orc_gemv_w4.argtypes = [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64]
        L.orc_gemm_w4.argtypes = [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64]
        L.orc_gemv_w4_f64.argtypes = [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64]
        L.orc_swiglu_h_w4.argtypes = [_vp] * 8 + [_i64, _i64, _i64]
        L.orc_swiglu_mlp_w4.argtypes = [_vp] * 11 + [_i64] * 5
        L.orc_swiglu_mlp_w4a8.argtypes = [_vp] * 11 + [_i64] * 4
        L.orc_gemv_w8.argtypes = [_vp, _vp, _vp, _i64, _vp, _vp, _i64, _i64]
        L.orc_quantize_int8.argtypes = [_f32p, _i8p, _f32p, _i64, _i64]
        L.orc_swiglu_h_w8.argtypes = [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _i64,
                                      _i64]
        L.orc_swiglu_mlp_w8.argtypes = [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp,
                                        _i64, _vp, _vp, _i64, _i64, _i64, _i64]
        L.orc_gemv_w4_rows.argtypes = [_vp, _vp, _vp, _i64, _vp, _vp, _i64, _i64]
        L.orc_quantize_int4_rows.argtypes = [_f32p, _u8p, _f32p, _i64, _i64]
        L.orc_rms_norm_torch.argtypes = [_f32p, _f32p, _f32p, _i64, C.c_float]
        L.orc_attention_layer.argtypes = [_f32p, _vp, _vp, _f32p, _i64, _i64, _i64, _i64, _i64]
        L.orc_decoder_set_rope_tables.argtypes = [_vp, _f32p, _f32p]
        L.orc_decoder_set_layer_path.argtypes = [_vp, C.c_int]
        L.orc_decoder_set_attention_cap.argtypes = [_vp, _i64]
        L.orc_decoder_set_a8.argtypes = [_vp, C.c_int]
        L.orc_rms_norm.argtypes = [_f32p, _f32p, _f32p, _i64, C.c_float]
        L.orc_gemv_f32.argtypes = [_vp, _vp, _vp, _i64, _i64]
        L.orc_rope_tables.argtypes = [_f32p, _f32p, _i64, _i64, C.c_double]
        L.orc_rope_apply.argtypes = [_f32p, _f32p, _f32p, _i64]
        L.orc_attention.argtypes = [_f32p, _vp, _vp, _f32p, _i64, _i64, _i64, _i64, _i64]
        L.orc_argmax.argtypes = [_f32p, _i64]
        L.orc_argmax.restype = _i64
        L.orc_decoder_create.argtypes = [_i64] * 9 + [C.c_double, C.c_float, C.c_int, C.c_int,
                                                      _vp, _vp, _vp, _vp]
        L.orc_decoder_create.restype = _vp
        L.orc_decoder_set_layer.argtypes = [_vp, _i64] + [_vp] * 13
        L.orc_decoder_destroy.argtypes = [_vp]
        L.orc_decoder_step.argtypes = [_vp, _i64, _i64]
        L.orc_decoder_logits.argtypes = [_vp]
        L.orc_decoder_logits.restype = C.POINTER(C.c_float)
        L.orc_decoder_k_cache.argtypes = [_vp, _i64]
        L.orc_decoder_k_cache.restype = C.POINTER(C.c_float)
        L.orc_decoder_v_cache.argtypes = [_vp, _i64]
        L.orc_decoder_v_cache.restype = C.POINTER(C.c_float)
        L.orc_decoder_kv_len.argtypes = [_vp]
        L.orc_decoder_kv_len.restype = _i64
        L.orc_decoder_copy_kv.argtypes = [_vp, _i64, _vp, _vp, _i64, _i64]
        L.orc_decoder_copy_kv.restype = C.c_int
        L.orc_num_threads.restype = C.c_int
        L.orc_set_num_threads.argtypes = [C.c_int]
        _u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16_n.argtypes = [_f32p, _u16p, _i64]
        L.orc_f16_to_f32_n.argtypes = [_u16p, _f32p, _i64]
        L.orc_pack_v1_to_v2.argtypes = [_u8p, _f32p, _u8p, _i64, _i64]
        L.orc_gemv_w4_v2.argtypes = [_vp, _vp, _vp, _vp, _i64, _i64]
        L.orc_gemm_w4_v2.argtypes = [_vp, _vp, _vp, _vp, _i64, _i64, _i64]
        L.orc_quantize_act_u8.argtypes = [_f32p, _i64, _u8p]
        L.orc_quantize_act_u8.restype = C.c_float
        L.orc_gemv_w4a8_g64.argtypes = [_vp, _vp, _vp, C.c_int, _vp, _vp, _i64, _i64]
        L.orc_repetition_penalty.argtypes = [_f32p, _i64, _vp, _i64, C.c_float]
        L.orc_sample_logits.argtypes = [_f32p, _i64, C.c_float, _i64, C.c_float, C.c_float,
                                        C.POINTER(_i64)]
        L.orc_sample_logits.restype = _i64
        L.orc_speculative_accept.argtypes = [_vp, _vp, _vp, _i64, _i64, C.c_float, C.c_float,
                                             _vp, _i64, C.POINTER(_i64), C.POINTER(_i64)]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dt):
    return None if a is None else np.ascontiguousarray(a, dtype=dt)


def num_threads() -> int:
    return int(lib().orc_num_threads())


def set_num_threads(n: int) -> None:
    """OpenMP threads of the oracle's parallel loops (the Rayon pool size)."""
    lib().orc_set_num_threads(int(n))


def pack_int4(q: np.ndarray) -> np.ndarray:
    q = _c(q, np.int8)
    n, k = q.shape
    out = np.empty((n, (k + 1) // 2), np.uint8)
    lib().orc_pack_int4(q, out, n, k)
    return out


def unpack_int4(w: np.ndarray, k: int) -> np.ndarray:
    w = _c(w, np.uint8)
    n = w.shape[0]
    out = np.empty((n, k), np.int8)
    lib().orc_unpack_int4(w, out, n, k)
    return out


def quantize_int4_grouped(w: np.ndarray, group_size: int):
    w = _c(w, np.float32)
    n, k = w.shape
    packed = np.empty((n, (k + 1) // 2), np.uint8)
    scales = np.empty((n, k // group_size), np.float32)
    lib().orc_quantize_int4_grouped(w, packed, scales, n, k, group_size)
    return packed, scales


def gemm_w4(x, w, s, bias=None, group_size=32) -> np.ndarray:
    """y[M, N] of the reference's gemm_w4a32_grouped (gemv.rs:1690-1725)."""
    x = _c(x, np.float32)
    w, s, bias = _c(w, np.uint8), _c(s, np.float32), _c(bias, np.float32)
    k = x.shape[-1]
    m = x.size // k
    n = w.shape[0]
    y = np.empty((m, n), np.float32)
    lib().orc_gemm_w4(_p(x), _p(w), _p(s), _p(bias), _p(y), m, n, k, group_size)
    return y.reshape(*x.shape[:-1], n)


def gemv_w4_f64(x, w, s, bias=None, group_size=32) -> np.ndarray:
    x = _c(x, np.float32).reshape(-1)
    w, s, bias = _c(w, np.uint8), _c(s, np.float32), _c(bias, np.float32)
    n = w.shape[0]
    y = np.empty(n, np.float64)
    lib().orc_gemv_w4_f64(_p(x), _p(w), _p(s), _p(bias), _p(y), n, x.size, group_size)
    return y


def f32_to_f16_bits(v) -> np.ndarray:
    """IEEE binary16 bits of each f32, round to nearest even (packed_v2.rs:66-105)."""
    v = _c(v, np.float32).reshape(-1)
    out = np.empty(v.size, np.uint16)
    lib().orc_f32_to_f16_n(v, out, v.size)
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    """binary16 bits -> f32 (packed_v2.rs:32-56)."""
    h = _c(h, np.uint16).reshape(-1)
    out = np.empty(h.size, np.float32)
    lib().orc_f16_to_f32_n(h, out, h.size)
    return out


def pack_v1_to_v2(w: np.ndarray, s: np.ndarray, k: int) -> np.ndarray:
    """v1 nibbles [n, k/2] + f32 scales [n, k/64] -> v2 blocks [n, (k/64) * 34]."""
    w, s = _c(w, np.uint8), _c(s, np.float32)
    n = w.shape[0]
    out = np.empty((n, (k // 64) * 34), np.uint8)
    lib().orc_pack_v1_to_v2(w, s, out, n, k)
    return out


def gemm_w4_v2(x, blocked, bias=None) -> np.ndarray:
    """w4a32_grouped_linear_v2 (packed_v2.rs:489-553), exact (non-VNNI) tiers."""
    x = _c(x, np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    m, k = x2.shape
    blocked = _c(blocked, np.uint8)
    n = blocked.shape[0]
    y = np.empty((m, n), np.float32)
    b = None if bias is None else _c(bias, np.float32)
    lib().orc_gemm_w4_v2(_p(x2), _p(blocked), _p(b), _p(y), m, n, k)
    return y


def quantize_act_u8(x):
    """(bytes, s_x) of quantize_activation_to_u8 (gemv.rs:1353-1389)."""
    x = _c(x, np.float32).reshape(-1)
    out = np.empty(x.size, np.uint8)
    sx = lib().orc_quantize_act_u8(x, x.size, out)
    return out, float(np.float32(sx))


def gemm_w4a8_g64(x, w, s=None, bias=None, blocked=False) -> np.ndarray:
    """The AVX-512 VNNI tier's W4A8 GEMV at group 64 (gemv.rs:1422-1473; v2 blocks
    packed_v2.rs:204-323), one activation row at a time."""
    x = _c(x, np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    m, k = x2.shape
    w = _c(w, np.uint8)
    n = w.shape[0]
    sv = None if s is None else _c(s, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    y = np.empty((m, n), np.float32)
    for i in range(m):
        xi = np.ascontiguousarray(x2[i])
        yi = np.empty(n, np.float32)
        lib().orc_gemv_w4a8_g64(_p(xi), _p(w), _p(sv), int(blocked), _p(b), _p(yi), n, k)
        y[i] = yi
    return y


def repetition_penalty(logits, recent, penalty) -> np.ndarray:
    """apply_repetition_penalty (decoder.rs:878-899) on a copy."""
    lg = np.array(logits, dtype=np.float32, copy=True).reshape(-1)
    rec = np.ascontiguousarray(np.asarray(list(recent), dtype=np.int64))
    lib().orc_repetition_penalty(lg, lg.size, rec.ctypes.data if rec.size else None, rec.size,
                                 float(penalty))
    return lg


def sample_logits(logits, temperature, top_k, top_p, u):
    """(token, candidates) of sample_logits (decoder.rs:908-1020) with the draw u."""
    lg = _c(logits, np.float32).reshape(-1)
    kept = _i64()
    tok = lib().orc_sample_logits(lg, lg.size, float(temperature), int(top_k), float(top_p),
                                  float(u), C.byref(kept))
    return int(tok), int(kept.value)


def speculative_accept(rows, draft, draft_probs, u, temperature=1.0, top_p=1.0):
    """(accepted, bonus) of speculative_accept's acceptance (decoder.rs:608-726)."""
    rows = _c(rows, np.float32)
    k, v = rows.shape
    d = np.ascontiguousarray(np.asarray(list(draft), dtype=np.int64))
    dp = _c(draft_probs, np.float32).reshape(-1)
    uu = np.ascontiguousarray(np.asarray(list(u), dtype=np.float64))
    a, b = _i64(), _i64()
    lib().orc_speculative_accept(_p(rows), _p(d), _p(dp), k, v, float(temperature), float(top_p),
                                 _p(uu) if uu.size else None, uu.size, C.byref(a), C.byref(b))
    return int(a.value), int(b.value)


def swiglu_mlp_w4(x, gw, gsc, uw, usc, dw, dsc, gb=None, ub=None, db=None, group_size=32):
    """fused_swiglu_mlp_w4a32 (fused_ops.rs:138-424); no residual."""
    x = _c(x, np.float32)
    k = x.shape[-1]
    m = x.size // k
    inter, nout = gw.shape[0], dw.shape[0]
    arrs = [_c(a, dt) for a, dt in ((gw, np.uint8), (gsc, np.float32), (gb, np.float32),
                                    (uw, np.uint8), (usc, np.float32), (ub, np.float32),
                                    (dw, np.uint8), (dsc, np.float32), (db, np.float32))]
    out = np.empty((m, nout), np.float32)
    lib().orc_swiglu_mlp_w4(_p(x), *[_p(a) for a in arrs], _p(out), m, k, inter, nout,
                            group_size)
    return out.reshape(*x.shape[:-1], nout)


def swiglu_mlp_w4a8(x, gw, gsc, uw, usc, dw, dsc, gb=None, ub=None, db=None):
    """fused_swiglu_mlp_w4a32 at group 64 on an AVX-512 VNNI host: W4A8 gate / up
    on x's bytes and W4A8 down on h's (fused_ops.rs:215-232, 409-421); no
    residual."""
    x = _c(x, np.float32)
    k = x.shape[-1]
    m = x.size // k
    inter, nout = gw.shape[0], dw.shape[0]
    arrs = [_c(a, dt) for a, dt in ((gw, np.uint8), (gsc, np.float32), (gb, np.float32),
                                    (uw, np.uint8), (usc, np.float32), (ub, np.float32),
                                    (dw, np.uint8), (dsc, np.float32), (db, np.float32))]
    out = np.empty((m, nout), np.float32)
    lib().orc_swiglu_mlp_w4a8(_p(x), *[_p(a) for a in arrs], _p(out), m, k, inter, nout)
    return out.reshape(*x.shape[:-1], nout)


def swiglu_h_w4(x, gw, gsc, uw, usc, gb=None, ub=None, group_size=32):
    x = _c(x, np.float32).reshape(-1)
    inter = gw.shape[0]
    h = np.empty(inter, np.float32)
    a = [_c(gw, np.uint8), _c(gsc, np.float32), _c(gb, np.float32), _c(uw, np.uint8),
         _c(usc, np.float32), _c(ub, np.float32)]
    lib().orc_swiglu_h_w4(_p(x), *[_p(t) for t in a], _p(h), inter, x.size, group_size)
    return h


def gemv_w8(x, w, s, bias=None) -> np.ndarray:
    """w8a32_linear (gemv.rs:974-1061), any number of x rows."""
    x = _c(x, np.float32)
    w, s, bias = _c(w, np.int8), _c(s, np.float32).reshape(-1), _c(bias, np.float32)
    k = x.shape[-1]
    m = x.size // k
    n = w.shape[0]
    y = np.empty((m, n), np.float32)
    xf = x.reshape(m, k)
    for i in range(m):
        row = np.ascontiguousarray(xf[i])
        lib().orc_gemv_w8(_p(row), _p(w), _p(s), s.size, _p(bias), y[i].ctypes.data, n, k)
    return y.reshape(*x.shape[:-1], n)


def gemv_w4_rows(x, w, s, bias=None, k=None) -> np.ndarray:
    """Per-channel w4a32_linear (gemv.rs:1066-1182), any number of x rows:
    y = dot_f32_u4(x, w_row) * s + b, s of 1 or N elements."""
    x = _c(x, np.float32)
    k = x.shape[-1] if k is None else k
    m = x.size // k
    w, s, bias = _c(w, np.uint8), _c(s, np.float32).reshape(-1), _c(bias, np.float32)
    n = w.shape[0]
    y = np.empty((m, n), np.float32)
    xf = x.reshape(m, k)
    for i in range(m):
        row = np.ascontiguousarray(xf[i])
        lib().orc_gemv_w4_rows(_p(row), _p(w), _p(s), s.size, _p(bias), y[i].ctypes.data, n, k)
    return y.reshape(*x.shape[:-1], n)


def quantize_int4_rows(w: np.ndarray):
    """quantize_linear_weights_int4 (fused_ops.rs:592-639): packed (N, ceil(K/2))
    and one scale per row."""
    w = _c(w, np.float32)
    n, k = w.shape
    q = np.empty((n, (k + 1) // 2), np.uint8)
    s = np.empty(n, np.float32)
    lib().orc_quantize_int4_rows(w, q, s, n, k)
    return q, s


def swiglu_h_w8(x, gw, gsc, uw, usc, gb=None, ub=None) -> np.ndarray:
    """The neuron loop of fused_swiglu_mlp_w8a32 (fused_ops.rs:71-113) for one
    token: scales of 1 element are per-tensor scalars, biases may be None."""
    x = _c(x, np.float32).reshape(-1)
    gw, uw = _c(gw, np.int8), _c(uw, np.int8)
    gsc, usc = _c(gsc, np.float32).reshape(-1), _c(usc, np.float32).reshape(-1)
    gb, ub = _c(gb, np.float32), _c(ub, np.float32)
    inter = gw.shape[0]
    h = np.empty(inter, np.float32)
    lib().orc_swiglu_h_w8(_p(x), _p(gw), _p(gsc), gsc.size, _p(gb), _p(uw), _p(usc), usc.size,
                          _p(ub), _p(h), inter, x.size)
    return h


def swiglu_mlp_w8(x, gw, gsc, uw, usc, dw, dsc, gb=None, ub=None, db=None) -> np.ndarray:
    """fused_swiglu_mlp_w8a32 (fused_ops.rs:8-133) over every row of x."""
    x = _c(x, np.float32)
    k = x.shape[-1]
    m = x.size // k
    gw, uw, dw = _c(gw, np.int8), _c(uw, np.int8), _c(dw, np.int8)
    gsc, usc, dsc = (_c(a, np.float32).reshape(-1) for a in (gsc, usc, dsc))
    gb, ub, db = _c(gb, np.float32), _c(ub, np.float32), _c(db, np.float32)
    inter, nout = gw.shape[0], dw.shape[0]
    out = np.empty((m, nout), np.float32)
    lib().orc_swiglu_mlp_w8(_p(x), _p(gw), _p(gsc), gsc.size, _p(gb), _p(uw), _p(usc), usc.size,
                            _p(ub), _p(dw), _p(dsc), dsc.size, _p(db), _p(out), m, k, inter, nout)
    return out.reshape(*x.shape[:-1], nout)


def quantize_int8(w: np.ndarray):
    w = _c(w, np.float32)
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    s = np.empty(n, np.float32)
    lib().orc_quantize_int8(w, q, s, n, k)
    return q, s


def rms_norm(x, w, eps) -> np.ndarray:
    x, w = _c(x, np.float32), _c(w, np.float32)
    out = np.empty_like(x)
    lib().orc_rms_norm(x, w, out, x.size, eps)
    return out


def rms_norm_torch(x, w, eps) -> np.ndarray:
    """F.rms_norm numerics of the per-layer Python path (model.py:91-98)."""
    x, w = _c(x, np.float32), _c(w, np.float32)
    out = np.empty_like(x)
    lib().orc_rms_norm_torch(x, w, out, x.size, eps)
    return out


def gemv_f32(x, w) -> np.ndarray:
    x, w = _c(x, np.float32).reshape(-1), _c(w, np.float32)
    y = np.empty(w.shape[0], np.float32)
    lib().orc_gemv_f32(_p(x), _p(w), _p(y), w.shape[0], w.shape[1])
    return y


def rope_tables(max_seq: int, head_dim: int, theta: float):
    c = np.empty((max_seq, head_dim), np.float32)
    s = np.empty((max_seq, head_dim), np.float32)
    lib().orc_rope_tables(c, s, max_seq, head_dim, theta)
    return c, s


def rope_apply(head, cos_row, sin_row) -> np.ndarray:
    h = np.array(head, dtype=np.float32, copy=True)
    lib().orc_rope_apply(h, _c(cos_row, np.float32), _c(sin_row, np.float32), h.size // 2)
    return h


def attention(q, k_cache, v_cache, seq_len: int) -> np.ndarray:
    """q [hq, hd]; caches [hkv, max_seq, hd]."""
    q = _c(q, np.float32)
    k_cache, v_cache = _c(k_cache, np.float32), _c(v_cache, np.float32)
    hq, hd = q.shape
    hkv, max_seq, _ = k_cache.shape
    out = np.empty_like(q)
    lib().orc_attention(q, _p(k_cache), _p(v_cache), out, hq, hkv, hd, max_seq, seq_len)
    return out


def attention_layer(q, k_cache, v_cache, seq_len: int) -> np.ndarray:
    """The per-layer steps' attention (fused_ops.rs:823-858, 997-1040)."""
    q = _c(q, np.float32)
    k_cache, v_cache = _c(k_cache, np.float32), _c(v_cache, np.float32)
    hq, hd = q.shape
    hkv, max_seq, _ = k_cache.shape
    out = np.empty_like(q)
    lib().orc_attention_layer(q, _p(k_cache), _p(v_cache), out, hq, hkv, hd, max_seq, seq_len)
    return out


def argmax(v) -> int:
    return int(lib().orc_argmax(_c(v, np.float32), np.asarray(v).size))


class Decoder:
    """The reference's RustQwenDecoder step (decoder.rs:1051-1374) on the CPU.

    Borrows the numpy weight arrays held in ``weights`` (kept alive here).
    wkind: 4 (INT4 grouped) or 8 (INT8 per-channel); lmkind: 4, 8 or 32 (fp32).
    rope_tables: (cos, sin) f32 [max_seq, head_dim] replacing the f64 tables.
    layer_path: the numerics of the reference's per-layer Python path
    (orc_decoder_set_layer_path), which runs INT8 and fp32-lm_head models.
    attention_cap: positions the native step scores (the reference's 32768,
    decoder.rs:1179-1184, unless a test sets another).
    a8: the W4A8 step of an AVX-512 VNNI host at group 64 (orc_decoder_set_a8).
    """

    def __init__(self, weights: dict, cfg: dict, rope_tables=None, layer_path=False,
                 attention_cap=32768, a8=False):
        self.cfg = cfg
        self.w = weights
        L = lib()
        lm_s = weights.get("lm_head_s")
        self.h = L.orc_decoder_create(
            cfg["num_layers"], cfg["hidden"], cfg["intermediate"], cfg["num_heads"],
            cfg["num_kv_heads"], cfg["head_dim"], cfg["vocab"], cfg["group_size"],
            cfg["max_seq"], float(cfg["rope_theta"]), float(cfg["eps"]), cfg["wkind"],
            cfg["lmkind"], _p(weights["embed"]), _p(weights["final_norm"]),
            _p(weights["lm_head_w"]), _p(lm_s))
        for li, lw in enumerate(weights["layers"]):
            L.orc_decoder_set_layer(
                self.h, li, _p(lw["in_norm"]), _p(lw["qkv_w"]), _p(lw["qkv_s"]), _p(lw["o_w"]),
                _p(lw["o_s"]), _p(lw["post_norm"]), _p(lw["gate_w"]), _p(lw["gate_s"]),
                _p(lw["up_w"]), _p(lw["up_s"]), _p(lw["down_w"]), _p(lw["down_s"]),
                _p(lw.get("qkv_b")))
        if rope_tables is not None:
            c, sn = (_c(t, np.float32) for t in rope_tables)
            assert c.shape == (cfg["max_seq"], cfg["head_dim"]) == sn.shape
            L.orc_decoder_set_rope_tables(self.h, c, sn)
        L.orc_decoder_set_layer_path(self.h, 1 if layer_path else 0)
        L.orc_decoder_set_attention_cap(self.h, int(attention_cap))
        L.orc_decoder_set_a8(self.h, 1 if a8 else 0)

    def step(self, token: int, offset: int) -> np.ndarray:
        L = lib()
        L.orc_decoder_step(self.h, token, offset)
        ptr = L.orc_decoder_logits(self.h)
        return np.ctypeslib.as_array(ptr, shape=(self.cfg["vocab"],)).copy()

    def copy_kv(self, layer: int, k: np.ndarray, v: np.ndarray, seq_len: int) -> None:
        k, v = _c(k, np.float32), _c(v, np.float32)
        rc = lib().orc_decoder_copy_kv(self.h, layer, _p(k), _p(v), k.shape[-2], seq_len)
        if rc != 0:
            raise ValueError("KV cache copy out of bounds")

    def kv_len(self) -> int:
        return int(lib().orc_decoder_kv_len(self.h))

    def close(self):
        if self.h:
            lib().orc_decoder_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

"""Loader for libtbhip.so and the status-code -> exception mapping.

The library is built in-tree by ``python -m torchburn_amd.build``.  There is no
CPU fallback: if the library or a GPU is missing, every op raises.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
# TB_LIB_SO: another build of the same sources (the host-sanitizer build of
# tests/run_sanitized.sh); by default the in-tree libtbhip.so
LIB_PATH = os.environ.get("TB_LIB_SO") or os.path.join(_HERE, "libtbhip.so")

TB_OK = 0
TB_ERR_UNSUPPORTED = 1
TB_ERR_VALUE = 2
TB_ERR_MEMORY = 3
TB_ERR_HIP = 4

UNSUPPORTED_MARKER = "TB_UNSUPPORTED:"


class UnsupportedOpError(RuntimeError):
    """Raised for shapes, dtypes or devices the kernels do not support.

    Mirrors the reference's UnsupportedOpError (src/dlpack.rs:35-53): a
    RuntimeError subclass whose message carries the "TB_UNSUPPORTED:" marker.
    """


_lock = threading.Lock()
_lib = None

_p = C.c_void_p
_i64 = C.c_int64

# name -> argtypes; every function returns int (status).
_SIGS = {
    "tb_w4a32_grouped_linear": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "tb_w4a32_grouped_linear_residual": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "tb_w4a32_grouped_linear_v2": [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "tb_pack_rows_w4a32_group64_v1_to_v2": [_p, _p, _p, _i64, _i64, _p],
    "tb_dequantize_int4_grouped_v2": [_p, _p, _i64, _i64, _p],
    "tb_set_vnni_semantics": [C.c_int],
    "tb_release_stream_workspace": [C.c_void_p],
    "tb_quantize_weight_int4_grouped": [_p, _p, _p, _i64, _i64, _i64, _p],
    "tb_quantize_weight_int8": [_p, _p, _p, _i64, _i64, _p],
    "tb_unpack_rows_w4a32_group64_v2_to_v1": [_p, _p, _p, _i64, _i64, _p],
    "tb_sample_logits": [_p, _i64, C.c_float, _i64, C.c_float, C.c_float, _p, _i64,
                         C.c_uint64, C.c_uint64, _p, _p, _p],
    "tb_swiglu_w4a32": [_p] * 8 + [_i64] * 4 + [_p],
    "tb_fused_swiglu_mlp_w4a32": [_p] * 12 + [_i64] * 5 + [_p],
    "tb_fused_swiglu_mlp_w4a32_noalloc": [_p] * 12 + [_i64] * 5 + [_p],
    "tb_w8a32_linear": [_p, _p, _p, _i64, _p, _p, _i64, _i64, _i64, _p],
    "tb_w4a32_linear": [_p, _p, _p, _i64, _p, _p, _i64, _i64, _i64, _p],
    "tb_quantize_weight_int4": [_p, _p, _p, _i64, _i64, _p],
    "tb_fused_swiglu_mlp_w8a32": [_p, _p, _p, _i64, _p, _p, _p, _i64, _p, _p, _p, _i64, _p, _p,
                                  _p] + [_i64] * 4 + [_p],
    "tb_xquant": [_p, _p, _i64, _i64, _p],
    "tb_read_probe": [_p, _i64, _i64, _i64, _p, _p, _p],
    "tb_w4a32_gemv_xq": [_p] * 7 + [_i64] * 4 + [_p],
    "tb_swiglu_w4a32_xq": [_p] * 9 + [_i64] * 4 + [_p],
    "tb_fused_attention_step_w4a32": [_p] * 12 + [_i64] * 7 + [_p],
    "tb_fused_attention_step_w8a32": [_p] * 3 + [_i64] + [_p] * 3 + [_i64] + [_p] * 6 +
                                     [_i64] * 6 + [_p],
    "tb_fused_transformer_layer_step_w4a32": [_p] * 22 + [_i64] * 8 + [C.c_double, _p],
}


def declared_symbols() -> list:
    """Every entry point the Python layer binds (all are declared in include/tbhip.h)."""
    return ["tb_last_error", "tb_version", "tb_x_records_bytes", "tb_sample_uniform",
            *_SIGS.keys()]


def lib():
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is missing; build it with `python -m torchburn_amd.build` "
                    "(there is no CPU fallback for the HIP path)")
            L = C.CDLL(LIB_PATH)
            L.tb_last_error.restype = C.c_char_p
            L.tb_version.restype = C.c_char_p
            L.tb_x_records_bytes.restype = C.c_int64
            L.tb_x_records_bytes.argtypes = [C.c_int64, C.c_int64]
            L.tb_sample_uniform.restype = C.c_float
            L.tb_sample_uniform.argtypes = [C.c_uint64, C.c_uint64]
            for name, args in _SIGS.items():
                fn = getattr(L, name)
                fn.argtypes = args
                fn.restype = C.c_int
            _lib = L
    return _lib


def check(rc: int) -> None:
    if rc == TB_OK:
        return
    msg = lib().tb_last_error().decode(errors="replace")
    if rc == TB_ERR_UNSUPPORTED:
        raise UnsupportedOpError(msg if UNSUPPORTED_MARKER in msg else f"{UNSUPPORTED_MARKER} {msg}")
    if rc == TB_ERR_VALUE:
        raise ValueError(msg)
    if rc == TB_ERR_MEMORY:
        raise MemoryError(msg)
    raise RuntimeError(f"HIP error: {msg}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))

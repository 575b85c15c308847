"""The C-ABI library (libtbhip.so): loads on a GPU-less host, exports every
entry point include/tbhip.h declares, and maps argument errors to the
reference's exception split without touching the GPU."""
import ctypes as C
import os
import re

import pytest

from torchburn_amd import _lib
from torchburn_amd import decoder as tbdec

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols(names=("tbhip.h", "tbhip_bench.h")):
    txt = "".join(open(os.path.join(ROOT, "include", n)).read() for n in names)
    return sorted(set(re.findall(r"TB_API\s+[\w\s\*]*?\b(tb_\w+)\s*\(", txt)))


def test_header_declares_entry_points():
    syms = header_symbols()
    assert "tb_w4a32_grouped_linear" in syms and "tb_decoder_step" in syms
    assert len(syms) >= 21
    # the measurement entry points stay out of the product header
    product = header_symbols(("tbhip.h",))
    assert "tb_read_probe" not in product and "tb_decoder_time_greedy" not in product
    assert "tbhip_bench.h" not in open(os.path.join(ROOT, "include", "tbhip.h")).read()


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for s in header_symbols():
        assert hasattr(L, s), s
    for s in _lib.declared_symbols() + tbdec.decoder_symbols():
        assert s in header_symbols(), s


def test_version_string():
    assert b"gfx950" in _lib.lib().tb_version()


def test_argument_errors_before_any_gpu_call():
    L = _lib.lib()
    buf = (C.c_float * 64)()
    p = C.cast(buf, C.c_void_p).value
    # an odd group size has no byte-aligned layout -> UnsupportedOpError
    rc = L.tb_w4a32_grouped_linear(p, p, p, None, p, 1, 1, 64, 9, None)
    assert rc == _lib.TB_ERR_UNSUPPORTED and b"even" in L.tb_last_error()
    with pytest.raises(_lib.UnsupportedOpError, match="TB_UNSUPPORTED"):
        _lib.check(rc)
    # negative dimension, null weight
    rc = L.tb_w4a32_grouped_linear(p, p, p, None, p, -1, 1, 64, 32, None)
    assert rc == _lib.TB_ERR_UNSUPPORTED
    rc = L.tb_w4a32_grouped_linear(p, None, p, None, p, 1, 1, 64, 32, None)
    assert rc == _lib.TB_ERR_UNSUPPORTED and b"null" in L.tb_last_error()
    # misaligned activations
    rc = L.tb_w4a32_grouped_linear(p + 2, p, p, None, p, 1, 1, 64, 32, None)
    assert rc == _lib.TB_ERR_UNSUPPORTED
    # per-channel scales: 1 or N elements
    rc = L.tb_w4a32_linear(p, p, p, 3, None, p, 1, 2, 64, None)
    assert rc == _lib.TB_ERR_UNSUPPORTED and b"1 or N" in L.tb_last_error()
    # INT8 MLP scale lengths (fused_ops.rs:80-97)
    rc = L.tb_fused_swiglu_mlp_w8a32(p, p, p, 5, None, p, p, 8, None, p, p, 8, None, None, p,
                                     1, 32, 8, 8, None)
    assert rc == _lib.TB_ERR_UNSUPPORTED and b"1 or N" in L.tb_last_error()
    # the read probe: loads per thread 4, 8 or 16; a 16-byte aligned buffer
    got = C.c_int64(0)
    rc = L.tb_read_probe(p, 1 << 20, 8, 5, p, C.addressof(got), None)
    assert rc == _lib.TB_ERR_UNSUPPORTED and b"loads" in L.tb_last_error()
    rc = L.tb_read_probe(p + 4, 1 << 20, 8, 4, p, C.addressof(got), None)
    assert rc == _lib.TB_ERR_UNSUPPORTED


@pytest.mark.parametrize("field,value,msg", [
    ("hidden_size", 898, "divisible by 4"),
    ("head_dim", 63, "even"),
    ("num_heads", 7, "divisible by num_kv_heads"),
    ("group_size", 48, "group_size"),
])
def test_decoder_config_errors_are_value_errors(field, value, msg):
    L = tbdec._bind()
    cfg = tbdec._Config(2, 256, 512, 4, 2, 64, 1000, 32, 128, 1e-6, 1e6, 4, 4)
    setattr(cfg, field, value)
    buf = (C.c_float * 16)()
    h = C.c_void_p()
    rc = L.tb_decoder_create(C.byref(cfg), buf, buf, buf, buf, C.byref(h))
    assert rc == _lib.TB_ERR_VALUE
    with pytest.raises(ValueError, match=msg):
        _lib.check(rc)


def test_product_path_never_touches_the_oracle():
    pkg = os.path.join(ROOT, "torchburn_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".cpp", ".h")):
                txt = open(os.path.join(dirpath, f)).read()
                for needle in ("import oracle", "from oracle", "liboracle", "orc_", "tb_oracle"):
                    assert needle not in txt, (f, needle)


def test_noalloc_scratch_limit_before_any_gpu_call():
    """tb_fused_swiglu_mlp_w4a32_noalloc checks the 16 MiB static scratch before
    any GPU work: the Llama-3-8B MLP (K 4096, I 14336) fits at M = 1..54 and
    65..88 and is refused with the byte count at M = 55..64 and from 89.  The
    pointers are placeholders: a shape that fits goes on to the device (none
    here) and fails with a HIP error, a refused one never gets there."""
    L = _lib.lib()
    A = C.c_void_p(1 << 20)   # 16-byte aligned, never dereferenced

    def call(m):
        return L.tb_fused_swiglu_mlp_w4a32_noalloc(A, A, A, None, A, A, None, A, A, None, None, A,
                                                   C.c_int64(m), C.c_int64(4096),
                                                   C.c_int64(14336), C.c_int64(4096),
                                                   C.c_int64(32), None)

    for m in (1, 8, 12, 16, 54, 65, 88):
        assert call(m) != _lib.TB_ERR_UNSUPPORTED, m
    for m in (55, 64, 89, 128):
        assert call(m) == _lib.TB_ERR_UNSUPPORTED, m
        assert b"static scratch holds 16777216" in L.tb_last_error()

"""Parity of the gfx950 INT4 GEMV / SwiGLU kernels with the CPU oracle.

The oracle (oracle/tb_oracle.c) restates the reference's gemv_w4a32_grouped
(src/quantization/gemv.rs:1514-1725) and fused_swiglu_mlp_w4a32
(src/quantization/fused_ops.rs:138-424).  Metric: max|d| / max|ref|, the
reference's own (tests/parity/int4.rs:131-141); bar 1e-4 (fp32 accumulate).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from torchburn_amd import synth
import torchburn_amd as tb

pytestmark = pytest.mark.gpu

TOL = 1e-4


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


SHAPES = [
    # (m, n, k, gs)
    (1, 4864, 896, 32),      # config 1 (Qwen2.5-0.5B MLP up-proj)
    (1, 64, 896, 64),        # the reference's own KAT shape (group 64)
    (1, 1152, 896, 32),      # Qwen qkv
    (1, 896, 4864, 32),      # Qwen down (K = 4864, 152 groups)
    (1, 14336, 4096, 32),    # Llama gate/up
    (1, 4096, 14336, 32),    # Llama down
    (2, 4096, 4096, 32),
    (3, 1000, 2048, 32),     # ragged N, odd M
    (4, 517, 1024, 64),
    (8, 4096, 4096, 32),     # config 2 batch 8
    (1, 7, 32, 32),          # one group per row
    (5, 33, 64, 32),
]


@pytest.mark.parametrize("m,n,k,gs", SHAPES)
def test_w4_linear_matches_oracle(cuda, m, n, k, gs):
    print(f"case w4a32_grouped_linear m={m} n={n} k={k} gs={gs}", flush=True)
    g = synth.rng(11, m, n, k, gs)
    x = synth.activations(g, m, k)
    w, s = synth.int4_weight(g, n, k, gs)
    bias = g.normal(0, 0.1, n).astype(np.float32)
    ref = O.gemm_w4(x, w, s, bias, group_size=gs)
    y = tb.w4a32_grouped_linear(torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda),
                                torch.from_numpy(s).to(cuda), torch.from_numpy(bias).to(cuda),
                                group_size=gs)
    torch.cuda.synchronize()
    assert rel(y.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("m,k,inter,gs", [(1, 896, 4864, 32), (1, 4096, 14336, 32),
                                          (4, 4096, 14336, 32), (8, 4096, 14336, 32),
                                          (2, 512, 1024, 64)])
def test_swiglu_mlp_residual_matches_oracle(cuda, m, k, inter, gs):
    print(f"case fused_swiglu_mlp m={m} k={k} inter={inter} gs={gs}", flush=True)
    g = synth.rng(12, m, k, inter)
    x = synth.activations(g, m, k)
    r = synth.activations(g, m, k)
    gw, gsc = synth.int4_weight(g, inter, k, gs)
    uw, usc = synth.int4_weight(g, inter, k, gs)
    dw, dsc = synth.int4_weight(g, k, inter, gs)
    ref = O.swiglu_mlp_w4(x, gw, gsc, uw, usc, dw, dsc, group_size=gs) + r
    T = lambda a: torch.from_numpy(a).to(cuda)
    out = tb.fused_swiglu_mlp_w4a32(T(x), T(gw), T(gsc), None, T(uw), T(usc), None, T(dw),
                                    T(dsc), None, group_size=gs, residual=T(r))
    torch.cuda.synchronize()
    assert rel(out.cpu().numpy(), ref) < TOL


def test_residual_in_place(cuda):
    g = synth.rng(13)
    x = synth.activations(g, 1, 4096)
    w, s = synth.int4_weight(g, 4096, 4096, 32)
    r = synth.activations(g, 1, 4096)
    ref = O.gemm_w4(x, w, s, None, group_size=32) + r
    T = lambda a: torch.from_numpy(a).to(cuda)
    rt = T(r)
    from torchburn_amd import _lib
    xt, wt, st = T(x), T(w), T(s)
    _lib.call("tb_w4a32_grouped_linear_residual", xt.data_ptr(), wt.data_ptr(), st.data_ptr(),
              None, rt.data_ptr(), rt.data_ptr(), 1, 4096, 4096, 32,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rel(rt.cpu().numpy(), ref) < TOL


def test_special_cases(cuda):
    """Closed forms: x == 0 -> bias; q == c with unit scales -> c * sum(x);
    one-hot x -> a column of the dequantized matrix."""
    n, k = 96, 256
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    bias = np.arange(n, dtype=np.float32)
    w = np.random.default_rng(0).integers(0, 256, (n, k // 2), dtype=np.uint8)
    s = np.ones((n, k // 32), np.float32)
    y = tb.w4a32_grouped_linear(T(np.zeros((1, k), np.float32)), T(w), T(s), T(bias), 32)
    assert np.array_equal(y.cpu().numpy()[0], bias)
    x = np.random.default_rng(1).standard_normal((1, k)).astype(np.float32)
    for c in (-8, -3, 0, 7):
        wc = np.full((n, k // 2), (c + 8) | ((c + 8) << 4), np.uint8)
        y = tb.w4a32_grouped_linear(T(x), T(wc), T(s), None, 32).cpu().numpy()[0]
        np.testing.assert_allclose(y, np.full(n, c * x.astype(np.float64).sum()), rtol=1e-5,
                                   atol=1e-4)
    s2 = np.random.default_rng(2).uniform(0.5, 2, (n, k // 32)).astype(np.float32)
    q = O.unpack_int4(w, k)
    for col in (0, 1, 31, 32, 255):
        e = np.zeros((1, k), np.float32)
        e[0, col] = 1.0
        y = tb.w4a32_grouped_linear(T(e), T(w), T(s2), None, 32).cpu().numpy()[0]
        np.testing.assert_array_equal(y, q[:, col].astype(np.float32) * s2[:, col // 32])


def test_errors_match_reference_contract(cuda):
    T = lambda a: torch.from_numpy(a).to(cuda)
    x = T(np.zeros((1, 64), np.float32))
    w = T(np.zeros((8, 31), np.uint8))
    s = T(np.ones((8, 2), np.float32))
    with pytest.raises(tb.UnsupportedOpError, match="TB_UNSUPPORTED"):
        tb.w4a32_grouped_linear(x, w, s, group_size=32)
    w = T(np.zeros((8, 32), np.uint8))
    with pytest.raises(tb.UnsupportedOpError, match="scales mismatch"):
        tb.w4a32_grouped_linear(x, w, T(np.ones((8, 3), np.float32)), group_size=32)
    # groups start on byte boundaries: an odd group size is refused, an even one
    # that the streaming kernels do not take runs the any-shape GEMV
    with pytest.raises(tb.UnsupportedOpError, match="group_size"):
        tb.w4a32_grouped_linear(x, w, T(np.ones((8, 8), np.float32)), group_size=9)
    g = synth.rng(15)
    xs = synth.activations(g, 1, 64)
    q = g.integers(-8, 8, (8, 64)).astype(np.int8)
    ss = (np.abs(g.normal(0, 0.02, (8, 4))) + 1e-3).astype(np.float32)
    y = tb.w4a32_grouped_linear(T(xs), T(O.pack_int4(q)), T(ss), group_size=16).cpu().numpy()
    assert rel(y, O.gemm_w4(xs, O.pack_int4(q), ss, None, group_size=16)) < TOL


def test_non_finite_activations_propagate(cuda):
    """NaN / Inf in x propagate as in the reference's f32 arithmetic."""
    g = synth.rng(14)
    n, k = 300, 4096
    w, s = synth.int4_weight(g, n, k, 32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    for bad in (np.nan, np.inf):
        x = synth.activations(g, 1, k)
        x[0, 1234] = bad
        ref = O.gemm_w4(x, w, s, None, group_size=32)
        y = tb.w4a32_grouped_linear(T(x), T(w), T(s), None, 32).cpu().numpy()
        assert np.array_equal(np.isnan(y), np.isnan(ref))
        assert np.array_equal(np.isinf(y), np.isinf(ref))
        fin = np.isfinite(ref)
        if fin.any():
            assert rel(y[fin], ref[fin]) < TOL


def test_extreme_activation_ranges(cuda):
    """Chunks mixing magnitudes 1e-30..1e30 and all-zero chunks."""
    g = synth.rng(15)
    n, k = 256, 2048
    w, s = synth.int4_weight(g, n, k, 32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    x = synth.activations(g, 1, k)
    x[0, :32] = 0.0
    x[0, 32:64] *= 1e-30
    x[0, 64:96] *= 1e30
    x[0, 100] = 1e20
    ref = O.gemm_w4(x, w, s, None, group_size=32)
    y = tb.w4a32_grouped_linear(T(x), T(w), T(s), None, 32).cpu().numpy()
    assert rel(y, ref) < TOL


@pytest.mark.parametrize("n,k,gs", [(4864, 896, 32), (4096, 14336, 32), (300, 2048, 64),
                                    (896, 4864, 32), (7, 64, 32)])
def test_in_kernel_records_match_prebuilt(cuda, n, k, gs):
    """One activation row of a single projection without x records: the GEMV
    builds each chunk's record from x itself.  Bit-identical to the same kernel
    fed the records of tb_xquant, including zero, tiny, huge and non-finite
    chunks."""
    from torchburn_amd import _lib
    print(f"case in-kernel records n={n} k={k} gs={gs}", flush=True)
    g = synth.rng(16, n, k, gs)
    x = synth.activations(g, 1, k)
    x[0, :32] = 0.0
    x[0, 32:48] *= 1e-33
    x[0, 48:64] *= 3e28
    x[0, k - 24:] = np.round(x[0, k - 24:] * 8) / 8   # exact small-step values
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    P = lambda t: t.data_ptr()
    S = torch.cuda.current_stream(cuda).cuda_stream
    w, s = synth.int4_weight(g, n, k, gs)
    b = g.normal(0, 0.1, n).astype(np.float32)
    r = synth.activations(g, 1, n)
    xt, wt, st, bt, rt = T(x), T(w), T(s), T(b), T(r)
    xq = torch.empty(_lib.lib().tb_x_records_bytes(1, k) // 4, dtype=torch.int32, device=cuda)
    want = torch.empty((1, n), device=cuda)

    def both():
        _lib.check(_lib.lib().tb_xquant(P(xt), P(xq), 1, k, S))
        _lib.check(_lib.lib().tb_w4a32_gemv_xq(P(xt), P(xq), P(wt), P(st), P(bt), P(rt),
                                               P(want), 1, n, k, gs, S))
        got = tb.w4a32_grouped_linear_residual(xt, wt, st, rt, bt, group_size=gs)
        torch.cuda.synchronize()
        return got.cpu().numpy(), want.cpu().numpy()

    gv, wv = both()
    np.testing.assert_array_equal(gv.view(np.uint32), wv.view(np.uint32))
    assert rel(gv, O.gemm_w4(x, w, s, b, group_size=gs) + r) < TOL
    # a NaN chunk reaches every output row on both paths
    x[0, k - 40] = np.nan
    xt.copy_(T(x))
    gv, wv = both()
    assert np.isnan(wv).all() and np.isnan(gv).all()

"""Parity of the batched INT4 projection (FP32 MFMA from M = 5) with the CPU oracle.

The oracle's gemm_w4 restates the reference's gemm_w4a32_grouped
(src/quantization/gemv.rs:1690-1725: one full GEMV per activation row), and
swiglu_mlp_w4 the batched SwiGLU of fused_swiglu_mlp_batched_w4a32
(src/quantization/fused_ops.rs:1267-1319).  Metric max|d| / max|ref|
(tests/parity/int4.rs:131-141), bar 1e-4.  Config 3: M in {16, 64}, K = 4096,
N in {4096, 14336}, group 32.
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


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


SHAPES = [
    # (m, n, k, gs)
    (16, 4096, 4096, 32),     # config 3
    (16, 14336, 4096, 32),    # config 3
    (64, 4096, 4096, 32),     # config 3
    (64, 14336, 4096, 32),    # config 3
    (15, 1000, 2048, 32),     # last GEMV row count
    (17, 1000, 2048, 32),     # ragged M and N
    (33, 517, 1024, 64),      # group 64, three M tiles
    (130, 96, 4096, 32),      # two M blocks of 64 plus a tail
    (16, 7, 32, 32),          # one group per row, N below a wave's 16 rows
    (20, 64, 96, 32),         # K not a multiple of the 128-wide step
    (48, 200, 192, 64),       # K = 1.5 steps, group 64
    (5, 4096, 4096, 32),      # verify-sized batches
    (8, 14336, 4096, 32),
    (7, 1000, 2048, 64),      # group 64
    (9, 517, 1024, 32),       # four-row tiles 3 of 4 used, ragged N
    (12, 96, 14336, 32),      # K split over many blocks
    (6, 33, 96, 32),          # 3 chunks, N below a wave's 16 rows
]


@pytest.mark.parametrize("m,n,k,gs", SHAPES)
def test_mfma_linear_matches_oracle(cuda, m, n, k, gs):
    print(f"case mfma w4a32_grouped_linear m={m} n={n} k={k} gs={gs}", flush=True)
    g = synth.rng(31, m, n, k, gs)
    x = synth.activations(g, m, k)
    w, s = synth.int4_weight(g, n, k, gs)
    bias = g.normal(0, 0.1, n).astype(np.float32)
    ref = O.gemm_w4(x, w, s, bias, group_size=gs)
    y = tb.w4a32_grouped_linear(T(x, cuda), T(w, cuda), T(s, cuda), T(bias, cuda), group_size=gs)
    torch.cuda.synchronize()
    err = rel(y.cpu().numpy(), ref)
    print(f"max rel err {err:.3g}", flush=True)
    assert err < TOL


# Up to 16 rows in shapes the small-batch limb path does not take (K % 128 != 0,
# or M = 16 with N, K <= 4096): the FP32-MFMA split-K projection, with and
# without the residual epilogue.
SMALL_M_SHAPES = [
    # (m, n, k, gs)
    (11, 300, 4064, 32),      # ragged N, K % 128 != 0
    (16, 4096, 1056, 32),     # 8.25 steps: the last K split ends inside a step
    (13, 77, 2112, 64),       # group 64
    (5, 2000, 160, 32),       # 2 steps
    (16, 4160, 4000, 32),     # N past 4096 with K % 128 != 0
    (16, 33, 4096, 128),      # group 128, one row block
]


@pytest.mark.parametrize("m,n,k,gs", SMALL_M_SHAPES)
def test_mfma_small_m_matches_oracle(cuda, m, n, k, gs):
    print(f"case mfma small-M m={m} n={n} k={k} gs={gs}", flush=True)
    g = synth.rng(35, m, n, k, gs)
    x = synth.activations(g, m, k)
    w, s = synth.int4_weight(g, n, k, gs)
    bias = g.normal(0, 0.1, n).astype(np.float32)
    r = synth.activations(g, m, n)
    ref = O.gemm_w4(x, w, s, bias, group_size=gs)
    y = tb.w4a32_grouped_linear(T(x, cuda), T(w, cuda), T(s, cuda), T(bias, cuda), group_size=gs)
    yr = tb.w4a32_grouped_linear_residual(T(x, cuda), T(w, cuda), T(s, cuda), T(r, cuda),
                                          T(bias, cuda), group_size=gs)
    torch.cuda.synchronize()
    err = rel(y.cpu().numpy(), ref)
    print(f"max rel err {err:.3g}", flush=True)
    assert err < TOL
    assert rel(yr.cpu().numpy(), ref + r) < TOL


def test_mfma_split_k_deterministic(cuda):
    """The K splits are summed in split order: repeated calls agree bit for bit."""
    g = synth.rng(36)
    m, n, k = 16, 4096, 4096
    x = T(synth.activations(g, m, k), cuda)
    w, s = synth.int4_weight(g, n, k, 32)
    w, s = T(w, cuda), T(s, cuda)
    ys = [tb.w4a32_grouped_linear(x, w, s, None, group_size=32).cpu().numpy() for _ in range(3)]
    assert np.array_equal(ys[0], ys[1]) and np.array_equal(ys[0], ys[2])


@pytest.mark.parametrize("m", [16, 64])
def test_mfma_residual_matches_oracle(cuda, m):
    print(f"case mfma residual m={m}", flush=True)
    g = synth.rng(32, m)
    n, k = 4096, 4096
    x = synth.activations(g, m, k)
    r = synth.activations(g, m, n)
    w, s = synth.int4_weight(g, n, k, 32)
    ref = O.gemm_w4(x, w, s, None, group_size=32) + r
    y = tb.w4a32_grouped_linear_residual(T(x, cuda), T(w, cuda), T(s, cuda), T(r, cuda),
                                         None, group_size=32)
    torch.cuda.synchronize()
    assert rel(y.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("m,k,inter,gs", [(16, 4096, 14336, 32), (64, 4096, 14336, 32),
                                          (24, 896, 4864, 32), (16, 512, 1024, 64),
                                          (12, 1056, 1120, 32),   # K % 128 != 0: FP32 MFMA
                                          (16, 2112, 3136, 64)])
def test_mfma_swiglu_mlp_matches_oracle(cuda, m, k, inter, gs):
    print(f"case mfma fused_swiglu_mlp m={m} k={k} inter={inter} gs={gs}", flush=True)
    g = synth.rng(33, m, k, inter)
    x = synth.activations(g, m, k)
    r = synth.activations(g, m, k)
    gw, gsc = synth.int4_weight(g, inter, k, gs)
    uw, usc = synth.int4_weight(g, inter, k, gs)
    dw, dsc = synth.int4_weight(g, k, inter, gs)
    gb = g.normal(0, 0.1, inter).astype(np.float32)
    ub = g.normal(0, 0.1, inter).astype(np.float32)
    ref = O.swiglu_mlp_w4(x, gw, gsc, uw, usc, dw, dsc, gb=gb, ub=ub, group_size=gs) + r
    out = tb.fused_swiglu_mlp_w4a32(T(x, cuda), T(gw, cuda), T(gsc, cuda), T(gb, cuda),
                                    T(uw, cuda), T(usc, cuda), T(ub, cuda), T(dw, cuda),
                                    T(dsc, cuda), None, group_size=gs, residual=T(r, cuda))
    torch.cuda.synchronize()
    err = rel(out.cpu().numpy(), ref)
    print(f"max rel err {err:.3g}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("shape", [(2, 40), (1, 1), (3, 1)])
def test_swiglu_mlp_batched_name_matches_oracle(cuda, shape):
    """fused_swiglu_mlp_batched_w4a32 on (batch, T, K): rows flattened, output
    (batch, T, N_down); no residual.  (1, 1) is the reference's per-token branch."""
    b, t = shape
    k, inter, gs = 896, 4864, 64
    print(f"case fused_swiglu_mlp_batched_w4a32 batch={b} T={t}", flush=True)
    g = synth.rng(34, b, t)
    x = synth.activations(g, b * t, k)
    gw, gsc = synth.int4_weight(g, inter, k, gs)
    uw, usc = synth.int4_weight(g, inter, k, gs)
    dw, dsc = synth.int4_weight(g, k, inter, gs)
    db = g.normal(0, 0.1, k).astype(np.float32)
    ref = O.swiglu_mlp_w4(x, gw, gsc, uw, usc, dw, dsc, db=db, group_size=gs)
    out = tb.fused_swiglu_mlp_batched_w4a32(T(x.reshape(b, t, k), cuda), T(gw, cuda),
                                            T(gsc, cuda), None, T(uw, cuda), T(usc, cuda), None,
                                            T(dw, cuda), T(dsc, cuda), T(db, cuda))
    torch.cuda.synchronize()
    assert tuple(out.shape) == (b, t, k)
    err = rel(out.cpu().numpy().reshape(b * t, k), ref)
    print(f"max rel err {err:.3g}", flush=True)
    assert err < TOL


def test_mfma_special_cases(cuda):
    """x == 0 -> bias exactly; one-hot rows -> columns of the dequantized matrix;
    constant q with unit scales -> c * sum(x)."""
    m, n, k = 16, 96, 256
    rng = np.random.default_rng(5)
    w = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    s = rng.uniform(0.5, 2, (n, k // 32)).astype(np.float32)
    bias = np.arange(n, dtype=np.float32)
    y = tb.w4a32_grouped_linear(T(np.zeros((m, k), np.float32), cuda), T(w, cuda), T(s, cuda),
                                T(bias, cuda), 32).cpu().numpy()
    assert np.array_equal(y, np.broadcast_to(bias, (m, n)))
    cols = [0, 1, 31, 32, 100, 127, 128, 255, 3, 64, 65, 200, 17, 18, 254, 129]
    e = np.zeros((m, k), np.float32)
    e[np.arange(m), cols] = 1.0
    y = tb.w4a32_grouped_linear(T(e, cuda), T(w, cuda), T(s, cuda), None, 32).cpu().numpy()
    q = O.unpack_int4(w, k)
    for i, c in enumerate(cols):
        np.testing.assert_array_equal(y[i], q[:, c].astype(np.float32) * s[:, c // 32])
    x = rng.standard_normal((m, k)).astype(np.float32)
    ones = np.ones((n, k // 32), np.float32)
    for c in (-8, 5):
        wc = np.full((n, k // 2), (c + 8) | ((c + 8) << 4), np.uint8)
        y = tb.w4a32_grouped_linear(T(x, cuda), T(wc, cuda), T(ones, cuda), None, 32).cpu().numpy()
        want = c * x.astype(np.float64).sum(axis=1, keepdims=True)
        np.testing.assert_allclose(y, np.broadcast_to(want, (m, n)), rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("m", [16, 6, 40, 70])
def test_mfma_non_finite_propagate(cuda, m):
    """NaN / Inf in one 16-row slab take the f32 path for that slab's batch
    (M = 40: the third slab of a block; M = 70: the fifth slab, a second block
    along M); the other slabs stay on the limbs."""
    g = synth.rng(34, m)
    n, k = 128, 1024
    w, s = synth.int4_weight(g, n, k, 32)
    x = synth.activations(g, m, k)
    x[3, 77] = np.nan
    x[m - 2, 500] = np.inf
    x[m - 2, 900] = -np.inf
    ref = O.gemm_w4(x, w, s, None, group_size=32)
    y = tb.w4a32_grouped_linear(T(x, cuda), T(w, cuda), T(s, cuda), None, 32).cpu().numpy()
    assert np.array_equal(np.isnan(y), np.isnan(ref))
    assert np.array_equal(np.isinf(y), np.isinf(ref))
    fin = np.isfinite(ref)
    assert rel(y[fin], ref[fin]) < TOL

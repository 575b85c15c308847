"""Parity of the small-batch INT4 projection (3..16 activation rows on f16
MFMA, csrc/w4_limb.hip) with the CPU oracle.

The oracle restates the reference's gemm_w4a32_grouped / w4a32_grouped_linear
(src/quantization/gemv.rs:1690-1725, packed_v2.rs:557-624), one GEMV per row,
its per-channel w4a32_linear (gemv.rs:1066-1182) and the batched SwiGLU MLP
(fused_ops.rs:1267-1319).  Metric max|d| / max|ref| per activation row (each
row of the batch is its own GEMV in the reference); bar 1e-4.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from torchburn_amd import synth
import torchburn_amd as tb

pytestmark = pytest.mark.gpu

TOL = 1e-4


def rel_rows(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    worst = 0.0
    for r in range(b.shape[0]):
        worst = max(worst, float(np.abs(a[r] - b[r]).max() / max(np.abs(b[r]).max(), 1e-30)))
    return worst


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("m,n,k,gs", [
    (3, 1000, 2048, 32), (7, 4096, 4096, 64), (8, 45, 256, 32),
    (9, 1000, 2048, 32), (12, 300, 1024, 128), (16, 4096, 4096, 32), (5, 14336, 4096, 32),
    (16, 1, 128, 32), (3, 33, 128, 64),
])
def test_limb_linear_matches_oracle(cuda, m, n, k, gs):
    print(f"case limb linear m={m} n={n} k={k} gs={gs}", flush=True)
    g = synth.rng(71, m, n, k, gs)
    x = synth.activations(g, m, k)
    w, s = synth.int4_weight(g, n, k, gs)
    b = g.normal(0, 0.1, n).astype(np.float32)
    ref = O.gemm_w4(x, w, s, b, group_size=gs)
    y = tb.w4a32_grouped_linear(T(x, cuda), T(w, cuda), T(s, cuda), T(b, cuda), group_size=gs)
    torch.cuda.synchronize()
    assert rel_rows(y.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("m", [4, 13])
def test_limb_residual(cuda, m):
    print(f"case limb residual m={m}", flush=True)
    g = synth.rng(72, m)
    n, k = 2048, 2048
    x = synth.activations(g, m, k)
    r = synth.activations(g, m, n)
    w, s = synth.int4_weight(g, n, k, 32)
    b = g.normal(0, 0.1, n).astype(np.float32)
    ref = O.gemm_w4(x, w, s, b, group_size=32) + r
    out = tb.w4a32_grouped_linear_residual(T(x, cuda), T(w, cuda), T(s, cuda), T(r, cuda),
                                           T(b, cuda), group_size=32)
    torch.cuda.synchronize()
    assert rel_rows(out.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("m,scalar", [(4, False), (12, True), (3, True)])
def test_limb_per_channel(cuda, m, scalar):
    """w4a32_linear with one scale per row or one scalar (gemv.rs:1114-1180)."""
    print(f"case limb w4a32_linear m={m} scalar={scalar}", flush=True)
    g = synth.rng(73, m, int(scalar))
    n, k = 777, 1024
    x = synth.activations(g, m, k)
    w = g.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    s = (np.abs(g.normal(0, 0.02, 1 if scalar else n)) + 1e-3).astype(np.float32)
    b = g.normal(0, 0.1, n).astype(np.float32)
    ref = O.gemv_w4_rows(x, w, s, b)
    y = tb.w4a32_linear(T(x, cuda), T(w, cuda), T(s, cuda), T(b, cuda)).cpu().numpy()
    assert rel_rows(y, ref) < TOL


@pytest.mark.parametrize("m,k,inter,gs", [(3, 1024, 2048, 32), (8, 4096, 14336, 32),
                                          (16, 1024, 2048, 64), (11, 512, 1024, 32),
                                          (4, 4096, 14336, 64)])
def test_limb_swiglu_mlp_with_biases(cuda, m, k, inter, gs):
    print(f"case limb MLP m={m} k={k} inter={inter} gs={gs}", flush=True)
    g = synth.rng(74, m, k, inter, gs)
    x = synth.activations(g, m, k)
    r = synth.activations(g, m, k)
    gw, gsc = synth.int4_weight(g, inter, k, gs)
    uw, usc = synth.int4_weight(g, inter, k, gs)
    dw, dsc = synth.int4_weight(g, k, inter, gs)
    gb = g.normal(0, 0.1, inter).astype(np.float32)
    ub = g.normal(0, 0.1, inter).astype(np.float32)
    db = g.normal(0, 0.1, k).astype(np.float32)
    ref = O.swiglu_mlp_w4(x, gw, gsc, uw, usc, dw, dsc, gb, ub, db, group_size=gs) + r
    out = tb.fused_swiglu_mlp_w4a32(T(x, cuda), T(gw, cuda), T(gsc, cuda), T(gb, cuda),
                                    T(uw, cuda), T(usc, cuda), T(ub, cuda), T(dw, cuda),
                                    T(dsc, cuda), T(db, cuda), group_size=gs,
                                    residual=T(r, cuda))
    torch.cuda.synchronize()
    assert rel_rows(out.cpu().numpy(), ref) < TOL


def test_limb_non_finite_propagate(cuda):
    """NaN / Inf rows: the flagged batches take the f32 path; other rows stay exact."""
    g = synth.rng(75)
    m, n, k = 6, 300, 2048
    w, s = synth.int4_weight(g, n, k, 32)
    x = synth.activations(g, m, k)
    x[1, 1234] = np.nan
    x[3, 77] = np.inf
    x[4, 500] = -np.inf
    ref = O.gemm_w4(x, w, s, None, group_size=32)
    y = tb.w4a32_grouped_linear(T(x, cuda), T(w, cuda), T(s, cuda), None, 32).cpu().numpy()
    assert np.array_equal(np.isnan(y), np.isnan(ref))
    assert np.array_equal(np.isinf(y), np.isinf(ref))
    assert np.array_equal(np.sign(y[np.isinf(ref)]), np.sign(ref[np.isinf(ref)]))
    fin = np.isfinite(ref).all(axis=1)
    assert fin[[0, 2, 5]].all()
    assert rel_rows(y[fin], ref[fin]) < TOL


def test_limb_extreme_ranges_and_zero_rows(cuda):
    """Groups spanning 1e-30..1e30, all-zero groups, an all-zero row, and a
    row above 2^100 (the f32 path)."""
    g = synth.rng(76)
    m, n, k = 5, 256, 2048
    w, s = synth.int4_weight(g, n, k, 32)
    b = g.normal(0, 0.1, n).astype(np.float32)
    x = synth.activations(g, m, k)
    x[0, :32] = 0.0
    x[0, 32:64] *= 1e-30
    x[0, 64:96] *= 1e30
    x[0, 100] = 1e20
    x[1] *= 1e-35
    x[2] = 0.0
    x[3, 640:672] *= 3e33
    ref = O.gemm_w4(x, w, s, b, group_size=32)
    y = tb.w4a32_grouped_linear(T(x, cuda), T(w, cuda), T(s, cuda), T(b, cuda), 32)
    y = y.cpu().numpy()
    np.testing.assert_array_equal(y[2], b)
    assert rel_rows(y, ref) < TOL


def test_limb_deterministic(cuda):
    g = synth.rng(77)
    m, n, k = 8, 4096, 4096
    x = T(synth.activations(g, m, k), cuda)
    w, s = synth.int4_weight(g, n, k, 32)
    w, s = T(w, cuda), T(s, cuda)
    y0 = tb.w4a32_grouped_linear(x, w, s, None, 32).cpu().numpy()
    y1 = tb.w4a32_grouped_linear(x, w, s, None, 32).cpu().numpy()
    np.testing.assert_array_equal(y0, y1)


def test_limb_whole_k_pair_partial_quad_and_nan(cuda):
    """The whole-K plan (records of all of K in LDS, one block per CU, no split)
    on a K of 31 batches (the last quad of batches is partial), with a NaN in
    one activation row: that token's outputs are NaN, the others match."""
    print("case limb whole-K MLP m=6 k=3968 inter=14336 + NaN row", flush=True)
    g = synth.rng(78)
    m, k, inter, gs = 6, 3968, 14336, 32
    x = synth.activations(g, m, k)
    gw, gsc = synth.int4_weight(g, inter, k, gs)
    uw, usc = synth.int4_weight(g, inter, k, gs)
    dw, dsc = synth.int4_weight(g, k, inter, gs)
    x[1, 2000] = np.nan
    ref = O.swiglu_mlp_w4(x, gw, gsc, uw, usc, dw, dsc, None, None, None, group_size=gs)
    out = tb.fused_swiglu_mlp_w4a32(T(x, cuda), T(gw, cuda), T(gsc, cuda), None,
                                    T(uw, cuda), T(usc, cuda), None, T(dw, cuda),
                                    T(dsc, cuda), None, group_size=gs)
    y = out.cpu().numpy()
    assert np.isnan(ref[1]).all() and np.isnan(y[1]).all()
    keep = [0, 2, 3, 4, 5]
    assert np.isfinite(y[keep]).all()
    assert rel_rows(y[keep], ref[keep]) < TOL


def test_limb_whole_k_single_projection(cuda):
    """A single projection with enough 16-row blocks for the whole-K plan."""
    print("case limb whole-K linear m=5 n=24576 k=4096", flush=True)
    g = synth.rng(79)
    m, n, k = 5, 24576, 4096
    w, s = synth.int4_weight(g, n, k, 32)
    b = g.normal(0, 0.1, n).astype(np.float32)
    x = synth.activations(g, m, k)
    ref = O.gemm_w4(x, w, s, b, group_size=32)
    y = tb.w4a32_grouped_linear(T(x, cuda), T(w, cuda), T(s, cuda), T(b, cuda), 32)
    assert rel_rows(y.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("m,k,inter,gs,bias", [
    (5, 4096, 14336, 32, True),    # whole-K pair, h only (no records for a next projection)
    (8, 4096, 12288, 32, False),   # whole-K pair at the plan's smallest size class
    (3, 4096, 10752, 64, True),    # whole-K pair, group-64 scales (one dword per group)
    (7, 2048, 14336, 128, False),  # whole-K pair, group 128, a short K
    (12, 2048, 4096, 32, True),    # two tiles: split partials and the pair reduce
    (3, 1024, 2048, 64, False),    # one tile, split partials
])
def test_limb_swiglu_pair_entry(cuda, m, k, inter, gs, bias):
    """tb_swiglu_w4a32, the neuron loop of fused_swiglu_mlp_w4a32
    (src/quantization/fused_ops.rs:244-407) on its own: h against the oracle."""
    from torchburn_amd import _lib
    print(f"case limb SwiGLU pair m={m} k={k} inter={inter} gs={gs} bias={bias}", flush=True)
    g = synth.rng(83, m, k, inter, gs)
    x = synth.activations(g, m, k)
    gw, gsc = synth.int4_weight(g, inter, k, gs)
    uw, usc = synth.int4_weight(g, inter, k, gs)
    gb = g.normal(0, 0.1, inter).astype(np.float32) if bias else None
    ub = g.normal(0, 0.1, inter).astype(np.float32) if bias else None
    ref = np.stack([O.swiglu_h_w4(x[r], gw, gsc, uw, usc, gb, ub, group_size=gs)
                    for r in range(m)])
    dx, dgw, dgs, duw, dus = (T(a, cuda) for a in (x, gw, gsc, uw, usc))
    dgb = T(gb, cuda) if bias else None
    dub = T(ub, cuda) if bias else None
    h = torch.full((m, inter), float("nan"), device=cuda)
    P = lambda t: t.data_ptr() if t is not None else None
    _lib.call("tb_swiglu_w4a32", P(dx), P(dgw), P(dgs), P(dgb), P(duw), P(dus), P(dub), P(h),
              m, k, inter, gs, torch.cuda.current_stream(cuda).cuda_stream)
    torch.cuda.synchronize(cuda)
    assert rel_rows(h.cpu().numpy(), ref) < TOL

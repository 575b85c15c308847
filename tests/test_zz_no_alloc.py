"""tb_fused_swiglu_mlp_w4a32_noalloc: the fused INT4 MLP with its intermediates
in the library's static device scratch (no allocation).  Called through the C
ABI and checked against tb_fused_swiglu_mlp_w4a32 (the same kernels on the
per-stream workspace) and the oracle, on two calls in a row, the second with a
smaller input; and the size limit."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from torchburn_amd import _lib, synth

pytestmark = pytest.mark.gpu


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def mlp_case(dev, seed, m, k, inter, gs):
    g = synth.rng(seed, m, k, inter)
    x = synth.activations(g, m, k)
    r = synth.activations(g, m, k)
    gw, gsc = synth.int4_weight(g, inter, k, gs)
    uw, usc = synth.int4_weight(g, inter, k, gs)
    dw, dsc = synth.int4_weight(g, k, inter, gs)
    ub = g.normal(0, 0.1, inter).astype(np.float32)
    ref = O.swiglu_mlp_w4(x, gw, gsc, uw, usc, dw, dsc, ub=ub, group_size=gs) + r
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return [T(a) for a in (x, gw, gsc, uw, usc, ub, dw, dsc, r)], ref


def call(name, t, m, k, inter, gs, dev):
    x, gw, gsc, uw, usc, ub, dw, dsc, r = t
    out = torch.empty((m, k), dtype=torch.float32, device=dev)
    P = lambda a: a.data_ptr()
    rc = getattr(_lib.lib(), name)(P(x), P(gw), P(gsc), None, P(uw), P(usc), P(ub), P(dw),
                                   P(dsc), None, P(r), P(out), m, k, inter, k, gs,
                                   torch.cuda.current_stream(dev).cuda_stream)
    return rc, out


def test_noalloc_matches_allocating_entry(cuda):
    # first Llama-3-8B MLPs at M = 16 and 8 (small-batch f16 MFMA; M = 16 needs
    # 11.3 MB of the 16 MiB scratch), then smaller ones at M = 3 (same path) and
    # M = 1 (the GEMV record path): the scratch keeps the previous call's
    # contents.
    for seed, m, k, inter in ((65, 16, 4096, 14336), (61, 8, 4096, 14336), (63, 3, 1024, 2048),
                              (62, 1, 1024, 2048)):
        print(f"case noalloc mlp m={m} k={k} inter={inter}", flush=True)
        t, ref = mlp_case(cuda, seed, m, k, inter, 32)
        rc, got = call("tb_fused_swiglu_mlp_w4a32_noalloc", t, m, k, inter, 32, cuda)
        _lib.check(rc)
        rc2, want = call("tb_fused_swiglu_mlp_w4a32", t, m, k, inter, 32, cuda)
        _lib.check(rc2)
        torch.cuda.synchronize()
        g, w = got.cpu().numpy(), want.cpu().numpy()
        assert rel(g, w) < 1e-6
        assert rel(g, ref) < 1e-4


def test_noalloc_rejects_oversized_scratch(cuda):
    # M = 64 runs the FP32-MFMA pair, whose split-K partials exceed the 16 MiB scratch
    m, k, inter = 64, 4096, 14336
    print(f"case noalloc size limit m={m} k={k} inter={inter}", flush=True)
    dev = cuda
    x = torch.zeros((m, k), device=dev)
    w = torch.zeros((inter, k // 2), dtype=torch.uint8, device=dev)
    s = torch.ones((inter, k // 32), device=dev)
    dw = torch.zeros((k, inter // 2), dtype=torch.uint8, device=dev)
    ds = torch.ones((k, inter // 32), device=dev)
    out = torch.empty((m, k), device=dev)
    P = lambda a: a.data_ptr()
    rc = _lib.lib().tb_fused_swiglu_mlp_w4a32_noalloc(
        P(x), P(w), P(s), None, P(w), P(s), None, P(dw), P(ds), None, None, P(out), m, k, inter,
        k, 32, torch.cuda.current_stream(dev).cuda_stream)
    assert rc == _lib.TB_ERR_UNSUPPORTED
    assert b"scratch" in _lib.lib().tb_last_error()


def test_noalloc_allocates_nothing(cuda):
    """Device memory is unchanged across a no-alloc call on a stream the library
    has never seen (a new stream would get a fresh workspace from the
    allocating entry).  The kernels are loaded first through the allocating
    entry, and the output is allocated before the measurement."""
    m, k, inter = 12, 4096, 14336
    print(f"case noalloc memory check m={m} k={k} inter={inter}", flush=True)
    t, ref = mlp_case(cuda, 66, m, k, inter, 32)
    rc, _ = call("tb_fused_swiglu_mlp_w4a32", t, m, k, inter, 32, cuda)
    _lib.check(rc)
    x, gw, gsc, uw, usc, ub, dw, dsc, r = t
    out = torch.empty((m, k), dtype=torch.float32, device=cuda)
    stream = torch.cuda.Stream(cuda)
    # A stream's first kernels make the HIP runtime and torch's caching
    # allocator set up per-stream memory of their own: a torch kernel on the
    # stream first, so that the measurement sees only the library's call.
    with torch.cuda.stream(stream):
        warm = torch.ones(1024, device=cuda) * 2
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info(cuda)[0]
    P = lambda a: a.data_ptr()
    rc = _lib.lib().tb_fused_swiglu_mlp_w4a32_noalloc(
        P(x), P(gw), P(gsc), None, P(uw), P(usc), P(ub), P(dw), P(dsc), None, P(r), P(out), m, k,
        inter, k, 32, stream.cuda_stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info(cuda)[0]
    assert free1 == free0, f"device memory changed by {free0 - free1} bytes"
    assert float(warm.sum()) == 2048.0
    assert rel(out.cpu().numpy(), ref) < 1e-4

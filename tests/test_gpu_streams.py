"""Stateless ops from several streams, threads and a captured graph.

The library keeps one scratch buffer per (device, stream) and never frees a
replaced one while the process lives (include/tbhip.h, workspace()).  The
reference allocates per call and runs concurrent GEMVs from 4 threads
(tests/test_audit_fixes.py:100-134); here every result is checked against the
oracle (max|d| / max|ref| < 1e-4).
"""
import threading

import numpy as np
import pytest
import torch

from oracle import oracle as O
from torchburn_amd import synth
import torchburn_amd as tb

pytestmark = pytest.mark.gpu


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def w4(g, n, k, gs=32):
    w, s = synth.int4_weight(g, n, k, gs)
    return w, s


def test_two_streams_interleaved(cuda):
    """A GEMV on one stream and a fused MLP on another, enqueued alternately with
    no synchronisation between them: each stream has its own records / h."""
    print("case two streams: w4a32_grouped_linear + fused_swiglu_mlp_w4a32", flush=True)
    g = synth.rng(51)
    K, N, I = 4096, 4096, 8192
    x1 = synth.activations(g, 1, K)
    w1, s1 = w4(g, N, K)
    x2 = synth.activations(g, 2, K)
    gw, gsc = w4(g, I, K)
    uw, usc = w4(g, I, K)
    dw, dsc = w4(g, K, I)
    ref1 = O.gemm_w4(x1, w1, s1, None, group_size=32)
    ref2 = O.swiglu_mlp_w4(x2, gw, gsc, uw, usc, dw, dsc, group_size=32)
    T = lambda a: torch.from_numpy(a).to(cuda)
    dx1, dw1, ds1 = T(x1), T(w1), T(s1)
    dx2, dgw, dgs, duw, dus, ddw, dds = (T(a) for a in (x2, gw, gsc, uw, usc, dw, dsc))
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    outs_a, outs_b = [], []
    for _ in range(12):
        with torch.cuda.stream(sa):
            outs_a.append(tb.w4a32_grouped_linear(dx1, dw1, ds1, None, group_size=32))
        with torch.cuda.stream(sb):
            outs_b.append(tb.fused_swiglu_mlp_w4a32(dx2, dgw, dgs, None, duw, dus, None, ddw,
                                                    dds, None, 32))
    torch.cuda.synchronize()
    for y in outs_a:
        assert rel(y.cpu().numpy(), ref1) < 1e-4
    for y in outs_b:
        assert rel(y.cpu().numpy(), ref2) < 1e-4


def test_four_threads_one_stream(cuda):
    """Four threads on the default stream, different x each (the reference's
    concurrency test pattern): the per-stream lease serialises their enqueues."""
    print("case four threads, default stream", flush=True)
    g = synth.rng(52)
    K, N = 2048, 1024
    w, s = w4(g, N, K)
    xs = [synth.activations(g, 1, K) for _ in range(4)]
    refs = [O.gemm_w4(x, w, s, None, group_size=32) for x in xs]
    dw, ds = torch.from_numpy(w).to(cuda), torch.from_numpy(s).to(cuda)
    dxs = [torch.from_numpy(x).to(cuda) for x in xs]
    torch.cuda.synchronize()
    errors, results = [], {}

    def worker(i):
        try:
            torch.cuda.set_device(cuda)
            outs = [tb.w4a32_grouped_linear(dxs[i], dw, ds, None, group_size=32)
                    for _ in range(10)]
            torch.cuda.synchronize()
            results[i] = [o.cpu().numpy() for o in outs]
        except Exception as e:   # reported below
            errors.append((i, e))

    th = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errors, errors
    for i in range(4):
        for y in results[i]:
            assert rel(y, refs[i]) < 1e-4


def test_quantized_linear_graph_capture(cuda):
    """A QuantizedLinear captured in a CUDA graph, then larger eager calls on the
    capture stream (its scratch grows and is replaced), then replays with new
    inputs: every replay matches the oracle."""
    print("case QuantizedLinear graph capture + larger call + replays", flush=True)
    torch.manual_seed(3)
    K, N = 2048, 1536
    q = tb.QuantizedLinear.from_float(torch.nn.Linear(K, N, bias=True), bits=4,
                                      group_size=32).to(cuda)
    wq, sq, bq = (t.detach().cpu().numpy() for t in (q.qweight, q.scales, q.bias))
    x_static = torch.randn(1, K, device=cuda)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        q(x_static)                    # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        y_static = q(x_static)
    gen = np.random.default_rng(4)
    for rep in range(4):
        with torch.cuda.stream(s):
            big = torch.randn(8 + 8 * rep, K, device=cuda)   # MFMA path, more scratch
            yb = q(big)
        torch.cuda.synchronize()
        assert rel(yb.cpu().numpy(),
                   O.gemm_w4(big.cpu().numpy(), wq, sq, bq, group_size=32)) < 1e-4
        xv = gen.standard_normal((1, K)).astype(np.float32)
        x_static.copy_(torch.from_numpy(xv))
        graph.replay()
        torch.cuda.synchronize()
        assert rel(y_static.cpu().numpy(), O.gemm_w4(xv, wq, sq, bq, group_size=32)) < 1e-4, rep


def test_capture_on_a_fresh_stream(cuda):
    """torch.cuda.graph on its own capture stream, never used before: the op's
    first call on that stream allocates its scratch during the capture; the
    replays match the oracle."""
    print("case capture on a fresh stream (scratch allocated under capture)", flush=True)
    g = synth.rng(53)
    K, I = 1024, 2048
    x = synth.activations(g, 1, K)
    gw, gsc = w4(g, I, K)
    uw, usc = w4(g, I, K)
    dw, dsc = w4(g, K, I)
    T = lambda a: torch.from_numpy(a).to(cuda)
    args = [T(a) for a in (gw, gsc)] + [None] + [T(a) for a in (uw, usc)] + [None] + \
        [T(a) for a in (dw, dsc)] + [None]
    dx = T(x)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):       # torch's capture stream, no warm-up on it
        y = tb.fused_swiglu_mlp_w4a32(dx, *args, 32)
    gen = np.random.default_rng(5)
    for rep in range(3):
        xv = gen.standard_normal((1, K)).astype(np.float32)
        dx.copy_(torch.from_numpy(xv))
        graph.replay()
        torch.cuda.synchronize()
        ref = O.swiglu_mlp_w4(xv, gw, gsc, uw, usc, dw, dsc, group_size=32)
        assert rel(y.cpu().numpy(), ref) < 1e-4, rep


def test_release_stream_workspace(cuda):
    """A stream's workspace is freed on request (device memory comes back) and a
    later call on the same stream gets a new one."""
    print("case release_stream_workspace", flush=True)
    g = synth.rng(57)
    K, I = 4096, 14336
    x = synth.activations(g, 8, K)
    gw, gsc = w4(g, I, K)
    uw, usc = w4(g, I, K)
    dw, dsc = w4(g, K, I)
    ref = O.swiglu_mlp_w4(x, gw, gsc, uw, usc, dw, dsc, group_size=32)
    T = lambda a: torch.from_numpy(a).to(cuda)
    args = [T(a) for a in (x, gw, gsc, uw, usc, dw, dsc)]
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        y1 = tb.fused_swiglu_mlp_w4a32(args[0], args[1], args[2], None, args[3], args[4], None,
                                       args[5], args[6], None, 32)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info(cuda)[0]
    tb.release_stream_workspace(s)
    free1 = torch.cuda.mem_get_info(cuda)[0]
    assert free1 > free0
    tb.release_stream_workspace(s)   # nothing left: a no-op
    with torch.cuda.stream(s):
        y2 = tb.fused_swiglu_mlp_w4a32(args[0], args[1], args[2], None, args[3], args[4], None,
                                       args[5], args[6], None, 32)
    torch.cuda.synchronize()
    assert rel(y1.cpu().numpy(), ref) < 1e-4 and rel(y2.cpu().numpy(), ref) < 1e-4

"""Benchmark of the gfx950 INT4 decode hot path (one MI355X).

Headline (BASELINE metric "INT4 GEMV HBM GB/s (% of 8 TB/s); decode tokens/sec
at 8B shape, 1 GPU"):

  * value: whole-step throughput of the Llama-3-8B-shape INT4 (group 32) SwiGLU
    MLP at batch M (default M = 1) through the public
    tb_fused_swiglu_mlp_w4a32: x records -> fused gate/up GEMV with silu*up
    (its epilogue also writes h's records) -> down GEMV with the residual add.
    One step = one pass over one synthetic activation row, weights resident in
    HBM.  Four distinct weight copies (4 x 110 MB > the 256 MB Infinity Cache)
    rotate, and the steps replay from one captured hipGraph, timed with HIP
    events on the capture stream.
  * roofline: the dominant kernel (fused gate/up GEMV, 73.5 MB per launch)
    timed alone the same way.
  * decode: Llama-3-8B INT4 (config 5), its INT8 repeat and Qwen2.5-0.5B with
    an fp32 lm_head (config 4): greedy steps as device-driven graph replays at
    KV length 4096 / 4096 / 2048, tokens/s and the fraction of the step's
    weight + KV byte roofline.
  * cpu_baseline: the C oracle (a restatement of the reference's CPU path) on
    this host's cores, on a bounded sample of the same MLP workload.

Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
MFMA_F32_PEAK = 157.3   # TFLOP/s, dense FP32 MFMA


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400, help="timed MLP steps")
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--m", type=int, default=1, help="activation rows (config 2: 1, 4, 8)")
    ap.add_argument("--copies", type=int, default=4, help="weight copies rotated (> 256 MB)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline budget")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-decode", default="llama4,qwen",
                    help="decode configs whose CPU-oracle tok/s is sampled, or 'none'")
    ap.add_argument("--no-config1", action="store_true", help="skip the config-1 GEMV line")
    ap.add_argument("--decode", default="llama4,llama8,qwen,qwen64",
                    help="decode runs: comma list of llama4, llama8, qwen, qwen64, or 'none'")
    ap.add_argument("--decode-steps", type=int, default=64)
    ap.add_argument("--prefill-tokens", type=int, default=512,
                    help="batched prefill timed on the llama4 decoder (0: skip)")
    ap.add_argument("--batched", default="16x4096,16x14336,64x4096,64x14336",
                    help="config 3 MxN projections (K=4096), or 'none'")
    ap.add_argument("--mlp-batches", default="4,8",
                    help="config 2 batch sizes M > 1 for the fused MLP, or 'none'")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (FETCH_SIZE / "
                         "WRITE_SIZE calibration for rocprofv3 --pmc), then exit")
    return ap.parse_args()


def cpu_info():
    """Host CPU facts for the baseline: model, SIMD flags, logical CPUs (nproc),
    physical cores, and the CPUs this process may run on (affinity)."""
    model, flags, cores = "", set(), set()
    phys = core = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and not model:
                    model = line.split(":", 1)[1].strip()
                if line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
                if line.startswith("physical id"):
                    phys = line.split(":", 1)[1].strip()
                if line.startswith("core id"):
                    core = line.split(":", 1)[1].strip()
                if not line.strip():
                    if core is not None:
                        cores.add((phys, core))
                    phys = core = None
            if core is not None:
                cores.add((phys, core))
    except OSError:
        pass
    keep = ("avx2", "fma", "avx512f", "avx512bw", "avx512_vnni")
    try:
        affinity = sorted(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = list(range(os.cpu_count() or 1))
    return dict(model=model, flags=sorted(f for f in flags if f in keep),
                nproc=os.cpu_count(), physical_cores=len(cores) or os.cpu_count(),
                affinity=f"{len(affinity)} CPUs: {affinity[0]}-{affinity[-1]}" if affinity else "")


PMC_SUMMARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                           "k_w4_gemv_swiglu_llama8b_mlp_m1_pmc.md")


def pmc_traffic():
    """HBM bytes per gate/up launch from the committed rocprofv3 --pmc summary:
    FETCH_SIZE and WRITE_SIZE (KiB per dispatch) times the scale factors that a
    plain copy kernel of known size gives for the same counters."""
    try:
        kv = {}
        with open(PMC_SUMMARY) as f:
            for line in f:
                if ":" in line and line.split(":")[0].strip() in (
                        "fetch_kib_per_dispatch", "write_kib_per_dispatch", "fetch_scale",
                        "write_scale"):
                    a, b = line.split(":", 1)
                    kv[a.strip()] = float(b)
        return int(round(1024 * (kv["fetch_kib_per_dispatch"] * kv["fetch_scale"] +
                                 kv["write_kib_per_dispatch"] * kv["write_scale"])))
    except (OSError, KeyError, ValueError):
        return None


def graph_time(torch, fn, reps, warmup, inner=1, spread=False):
    """Capture `inner` back-to-back calls of fn() as one graph, replay it `reps`
    times; returns ms per fn() call.  A graph replay costs a few microseconds
    of its own at its start and end, so short kernels are timed with enough of
    them per replay that this stays a small share of each.  spread: also
    returns the per-replay ms per call (one event pair around each replay)."""
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        fn()                      # allocate workspaces outside the capture
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(inner):
            fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    ev[0].record()
    for i in range(reps):
        g.replay()
        if spread:
            ev[i + 1].record()
    if not spread:
        ev[reps].record()
    torch.cuda.synchronize()
    ms = ev[0].elapsed_time(ev[reps]) / (reps * inner)
    if spread:
        per = [ev[i].elapsed_time(ev[i + 1]) / inner for i in range(reps)]
        return ms, g, per
    return ms, g


INNER = 10   # rotations of the weight copies per captured graph (MLP and GEMV timing)

# Grid shapes the read probe tries: (blocks of 256 threads, 16-byte loads in
# flight per thread).
PROBE_SHAPES = [(512, 4), (768, 4), (1024, 8), (1536, 4), (2048, 8)]


def read_ceiling(torch, dev, sizes, copies, reps, inner):
    """The fastest plain read (tb_read_probe: non-temporal 16-byte loads, no
    compute) of each byte count in `sizes`, over `copies` cold buffers rotated
    as the GEMV timing rotates its weight copies: what a read of the same bytes
    reaches on this GPU, to set each GEMV's bandwidth beside the 8 TB/s
    peak."""
    from torchburn_amd import _lib
    import ctypes
    big = max(sizes.values())
    buf = torch.empty(copies * big, dtype=torch.uint8, device=dev)
    buf.fill_(3)
    out = torch.empty(max(b for b, _ in PROBE_SHAPES) * 256, dtype=torch.int32, device=dev)
    S = lambda: torch.cuda.current_stream(dev).cuda_stream
    res = {}
    for name, nbytes in sizes.items():
        best = None
        for blocks, loads in PROBE_SHAPES:
            got = ctypes.c_int64(0)

            def reads():
                for c in range(copies):
                    _lib.call("tb_read_probe", buf.data_ptr() + c * big, nbytes, blocks, loads,
                              out.data_ptr(), ctypes.addressof(got), S())

            ms, _ = graph_time(torch, reads, reps, 1, inner)
            us = ms * 1e3 / copies
            gbs = got.value / (us * 1e-6) / 1e9
            if best is None or gbs > best["gbs"]:
                best = {"bytes": nbytes, "bytes_read": got.value, "us": round(us, 3),
                        "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                        "blocks": blocks, "loads_per_thread": loads}
        res[name] = best
    del buf
    return res


def mlp_section(torch, args, dev):
    from torchburn_amd import _lib
    M, K, I, GS = args.m, 4096, 14336, 32
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x7B + 2)

    def int4(n, k):
        w = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=dev, generator=gen)
        s = torch.randn((n, k // GS), device=dev, generator=gen).mul_(0.02).abs_().add_(1e-3)
        return w, s

    sets = [(*int4(I, K), *int4(I, K), *int4(K, I)) for _ in range(args.copies)]
    x = torch.randn((M, K), device=dev, generator=gen)
    r = torch.randn((M, K), device=dev, generator=gen)
    out = torch.empty((M, K), device=dev)
    h = torch.empty((M, I), device=dev)
    xq = torch.empty(_lib.lib().tb_x_records_bytes(M, K) // 4, dtype=torch.int32, device=dev)
    hq = torch.empty(_lib.lib().tb_x_records_bytes(M, I) // 4, dtype=torch.int32, device=dev)
    P = lambda t: t.data_ptr()
    S = lambda: torch.cuda.current_stream(dev).cuda_stream

    def mlp(ws):
        # The public fused entry point (reference fused_swiglu_mlp_w4a32 plus the
        # residual add): x records -> gate/up + silu*up (+ h records) -> down + r.
        gw, gs, uw, us, dw, ds = ws
        _lib.call("tb_fused_swiglu_mlp_w4a32", P(x), P(gw), P(gs), None, P(uw), P(us), None,
                  P(dw), P(ds), None, P(r), P(out), M, K, I, K, GS, S())

    def all_steps():
        for ws in sets:
            mlp(ws)

    # One replay = `inner` rotations of the copies (inner * copies MLP steps).
    inner = max(1, min(INNER, args.steps // len(sets)))
    per = inner * len(sets)
    reps = max(1, args.steps // per)
    ms_graph, _, per_rep = graph_time(torch, all_steps, reps, max(1, -(-args.warmup // per)),
                                      inner, spread=True)
    ms = ms_graph / len(sets)
    per_step = sorted(v / len(sets) for v in per_rep)
    timed_steps = reps * per
    w_bytes = 3 * (I * K // 2 + 4 * I * (K // GS))
    act_bytes = 4 * (M * K + 2 * M * I + 2 * M * K)
    step_bytes = w_bytes + act_bytes

    # Dominant kernel alone: fused gate/up GEMV over the rotation (records prebuilt).
    _lib.call("tb_xquant", P(x), P(xq), M, K, S())
    _lib.call("tb_xquant", P(h), P(hq), M, I, S())

    def gateups():
        for gw, gs, uw, us, _, _ in sets:
            _lib.call("tb_swiglu_w4a32_xq", P(x), P(xq), P(gw), P(gs), None, P(uw), P(us), None,
                      P(h), M, K, I, GS, S())

    def downs():
        for _, _, _, _, dw, ds in sets:
            _lib.call("tb_w4a32_gemv_xq", P(h), P(hq), P(dw), P(ds), None, P(r), P(out), M, K,
                      I, GS, S())

    gu_ms, _ = graph_time(torch, gateups, reps, 1, inner)
    dn_ms, _ = graph_time(torch, downs, reps, 1, inner)
    gu_us = gu_ms * 1e3 / len(sets)
    dn_us = dn_ms * 1e3 / len(sets)
    gu_bytes = 2 * (I * K // 2 + 4 * I * (K // GS)) + 4 * M * K + 4 * M * I
    dn_bytes = K * I // 2 + 4 * K * (I // GS) + 4 * M * I + 8 * M * K
    ceiling = read_ceiling(torch, dev, {"gate_up": 2 * (I * K // 2 + 4 * I * (K // GS)),
                                        "down": K * I // 2 + 4 * K * (I // GS)},
                           len(sets), reps, inner)

    # Parity guard on the measured data against the CPU oracle (set 0).
    from oracle import oracle as O
    torch.cuda.synchronize()
    mlp(sets[0])
    torch.cuda.synchronize()
    ws = [t.cpu().numpy() for t in sets[0]]
    xs, rs = x.cpu().numpy(), r.cpu().numpy()
    ref = O.swiglu_mlp_w4(xs, ws[0], ws[1], ws[2], ws[3], ws[4], ws[5], group_size=GS) + rs
    max_rel = float(np.abs(out.cpu().numpy() - ref).max() / np.abs(ref).max())

    cpu = None
    if not args.no_cpu:
        info = cpu_info()
        threads = info["physical_cores"]   # the reference's default pool size
        O.set_num_threads(threads)
        n, t0 = 0, time.perf_counter()
        while True:
            O.swiglu_mlp_w4(xs, ws[0], ws[1], ws[2], ws[3], ws[4], ws[5], group_size=GS)
            n += 1
            el = time.perf_counter() - t0
            if el > args.cpu_seconds:
                break
        cpu = {"value": round(step_bytes * n / el / 1e9, 3), "unit": "GB/s",
               "cores": O.num_threads(), "kind": "port",
               "sample": f"{n} M={M} MLP passes of the C oracle (restated reference CPU path) "
                         f"in {el:.1f} s",
               "ms_per_step": round(el / n * 1e3, 3),
               "host": info}
    del sets
    return dict(ms=ms, step_bytes=step_bytes, gu_us=gu_us, gu_bytes=gu_bytes, dn_us=dn_us,
                ceiling=ceiling,
                dn_bytes=dn_bytes, max_rel=max_rel, cpu=cpu, steps=timed_steps,
                spread={"replays": len(per_step),
                        "median_ms_per_step": round(per_step[len(per_step) // 2], 5),
                        "min_ms_per_step": round(per_step[0], 5),
                        "max_ms_per_step": round(per_step[-1], 5)})


def int4_set(torch, dev, gen, n, k, gs=32):
    w = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=dev, generator=gen)
    s = torch.randn((n, k // gs), device=dev, generator=gen).mul_(0.02).abs_().add_(1e-3)
    return w, s


def batched_kernel(M, N, K):
    """The kernel tb_w4a32_grouped_linear runs for an M x N x K v1 g32
    projection (the selection in csrc/capi.hip linear_w4 and csrc/w4_mfma.hip
    w4_mfma): M = 3..16 takes the small-batch f16-MFMA limb kernel (exact
    products from f16 limbs of x), except M = 16 with N and K at most 4096,
    which stays on FP32 MFMA; from M = 17 (K a multiple of 128) the batched
    limb GEMM.  Every entry's frac_fp32_mfma_peak is its f32-contraction rate
    over the FP32-MFMA peak; the limb kernels get there on f16 MFMA."""
    if 3 <= M <= 16 and not (M == 16 and N <= 4096 and K <= 4096):
        return "k_limb_prep + k_w4_limb (f16 MFMA on exact limbs of x) + k_limb_reduce"
    if M >= 17 and K % 128 == 0:
        return "k_lgemm_prep + k_w4_lgemm (f16 MFMA on exact limbs of x, 16-row slabs) + k_mfma_reduce"
    return "k_w4_mfma (FP32 MFMA) + k_mfma_reduce"


def batched_section(torch, args, dev):
    """Config 3: Y[M, N] = X[M, 4096] . deq(W)^T, M in {16, 64}."""
    from torchburn_amd import _lib
    K, GS = 4096, 32
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x7B + 3)
    out = {}
    S = lambda: torch.cuda.current_stream(dev).cuda_stream
    for spec in args.batched.split(","):
        M, N = (int(v) for v in spec.split("x"))
        copies = max(4, -(-300 * 2**20 // (N * K * 5 // 8)))   # > 256 MB of weights rotate
        sets = [int4_set(torch, dev, gen, N, K, GS) for _ in range(copies)]
        x = torch.randn((M, K), device=dev, generator=gen)
        y = torch.empty((M, N), device=dev)

        def run():
            for w, s in sets:
                _lib.call("tb_w4a32_grouped_linear", x.data_ptr(), w.data_ptr(), s.data_ptr(),
                          None, y.data_ptr(), M, N, K, GS, S())

        reps = 20
        ms, _ = graph_time(torch, run, reps, 3)
        us = ms * 1e3 / len(sets)
        flops = 2.0 * M * N * K
        wbytes = N * K // 2 + 4 * N * (K // GS)
        out[f"m{M}_n{N}"] = {"kernel": batched_kernel(M, N, K),
                             "us": round(us, 3), "tflops": round(flops / us / 1e6, 2),
                             "frac_fp32_mfma_peak": round(flops / us / 1e6 / MFMA_F32_PEAK, 4),
                             "weight_gbs": round(wbytes / us / 1e3, 1),
                             "weight_copies_rotated": copies}
        del sets
    torch.cuda.empty_cache()
    return out


def mlp_batch_section(torch, args, dev):
    """Config 2 at M > 1: the fused SwiGLU MLP with residual through the public
    entry point, 4 rotating weight copies; GB/s of the weight + activation bytes."""
    from torchburn_amd import _lib
    K, I, GS = 4096, 14336, 32
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x7B + 2)
    sets = [(*int4_set(torch, dev, gen, I, K), *int4_set(torch, dev, gen, I, K),
             *int4_set(torch, dev, gen, K, I)) for _ in range(4)]
    S = lambda: torch.cuda.current_stream(dev).cuda_stream
    out = {}
    for M in (int(v) for v in args.mlp_batches.split(",")):
        x = torch.randn((M, K), device=dev, generator=gen)
        r = torch.randn((M, K), device=dev, generator=gen)
        o = torch.empty((M, K), device=dev)

        def run():
            for gw, gs, uw, us, dw, ds in sets:
                _lib.call("tb_fused_swiglu_mlp_w4a32", x.data_ptr(), gw.data_ptr(), gs.data_ptr(),
                          None, uw.data_ptr(), us.data_ptr(), None, dw.data_ptr(), ds.data_ptr(),
                          None, r.data_ptr(), o.data_ptr(), M, K, I, K, GS, S())

        # the median of 20 replays of 20 steps each (the first configuration
        # measured otherwise read a few us slow on some boxes)
        _, _, per = graph_time(torch, run, 20, 3, 5, spread=True)
        us = statistics.median(per) * 1e3 / len(sets)
        byts = 3 * (I * K // 2 + 4 * I * (K // GS)) + 4 * (M * K + 2 * M * I + 2 * M * K)
        out[f"m{M}"] = {"us": round(us, 3), "gbs": round(byts / us / 1e3, 1),
                        "tok_s": round(M / us * 1e6, 1),
                        "us_min_max": [round(min(per) * 1e3 / len(sets), 3),
                                       round(max(per) * 1e3 / len(sets), 3)]}
    del sets
    torch.cuda.empty_cache()
    return out


def config1_line(torch, dev):
    """BASELINE config 1 (report only): one INT4 g32 GEMV, Qwen2.5-0.5B up-proj
    shape [4864, 896], M = 1, through tb_w4a32_grouped_linear (x records + GEMV),
    over > 256 MB of rotating weight copies."""
    from torchburn_amd import _lib
    N, K, GS = 4864, 896, 32
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x7B + 1)
    wbytes = N * K // 2 + 4 * N * (K // GS)
    copies = -(-300 * 2**20 // wbytes)
    sets = [int4_set(torch, dev, gen, N, K, GS) for _ in range(copies)]
    x = torch.randn((1, K), device=dev, generator=gen)
    y = torch.empty((1, N), device=dev)
    S = lambda: torch.cuda.current_stream(dev).cuda_stream

    def run():
        for w, sc in sets:
            _lib.call("tb_w4a32_grouped_linear", x.data_ptr(), w.data_ptr(), sc.data_ptr(), None,
                      y.data_ptr(), 1, N, K, GS, S())

    ms, _ = graph_time(torch, run, 5, 1)
    us = ms * 1e3 / len(sets)
    byts = wbytes + 4 * (K + N)
    del sets
    torch.cuda.empty_cache()
    return {"workload": "config 1: INT4 g32 GEMV [4864, 896], M=1 (report only)", "us": round(us, 3),
            "gbs": round(byts / us / 1e3, 1), "frac_hbm_peak": round(byts / us / 1e3 / HBM_PEAK_GBS, 4),
            "weight_copies_rotated": copies}


def cpu_decode(name):
    """The C oracle's decode step (the restated reference CPU decoder) for a
    decode config, on a bounded sample: a decoder of 2 layers of the real shape
    over the real KV length (greedy steps) and the lm_head GEMV alone; the
    per-layer time (2-layer step minus lm_head, halved) x the layer count plus
    the lm_head gives the full model's time per token."""
    from oracle import oracle as O
    from torchburn_amd import synth
    cfg, wk, lk, kvlen, seed = {
        "llama4": (synth.LLAMA3_8B, 4, 4, 4096, 0x7B + 5),
        "llama8": (synth.LLAMA3_8B, 8, 8, 4096, 0x7B + 5),
        "qwen": (synth.QWEN_0_5B, 4, 32, 2048, 0x7B + 4),
    }[name]
    info = cpu_info()
    O.set_num_threads(info["physical_cores"])
    c = dict(cfg, num_layers=2)
    w = synth.decoder_weights(c, seed, wk, lk, 32)
    max_seq = kvlen + 8
    dec = O.Decoder(w, dict(c, group_size=32, max_seq=max_seq, wkind=wk, lmkind=lk))
    for li, (k, v) in enumerate(synth.kv_prefill(c, seed, kvlen, max_seq)):
        dec.copy_kv(li, k, v, kvlen)
    tok = seed % cfg["vocab"]
    dec.step(tok, kvlen)                          # warm-up: touches every page once
    steps = []
    for i in range(1, 6):
        t0 = time.perf_counter()
        dec.step(tok, kvlen + i)
        steps.append(time.perf_counter() - t0)
    xn = np.random.default_rng(1).standard_normal((1, cfg["hidden"])).astype(np.float32)
    lm = []
    for _ in range(5):
        t0 = time.perf_counter()
        if lk == 4:
            O.gemm_w4(xn, w["lm_head_w"], w["lm_head_s"], None, group_size=32)
        elif lk == 8:
            O.gemv_w8(xn, w["lm_head_w"], w["lm_head_s"])
        else:
            O.gemv_f32(xn[0], w["lm_head_w"])
        lm.append(time.perf_counter() - t0)
    dec.close()
    t2, t_lm = min(steps), min(lm)
    t_layer = max(t2 - t_lm, 0.0) / 2
    t_tok = cfg["num_layers"] * t_layer + t_lm
    return {"tok_s": round(1.0 / t_tok, 3), "ms_per_token": round(t_tok * 1e3, 2),
            "cores": O.num_threads(), "kind": "port",
            "sample": f"oracle decoder of 2 {name} layers at KV {kvlen} (best of 5 steps "
                      f"{t2 * 1e3:.1f} ms) and its lm_head alone (best of 5, {t_lm * 1e3:.1f} ms); "
                      f"per-layer time x {cfg['num_layers']} layers + lm_head",
            "host": info}


def decode_run(torch, name, steps, prefill_tokens=0):
    from torchburn_amd import synth
    from torchburn_amd.decoder import decoder_from_weights
    cfg, wk, lk, kvlen, seed = {
        "llama4": (synth.LLAMA3_8B, 4, 4, 4096, 0x7B + 5),
        "llama8": (synth.LLAMA3_8B, 8, 8, 4096, 0x7B + 5),
        "qwen": (synth.QWEN_0_5B, 4, 32, 2048, 0x7B + 4),
        # the reference's own Qwen decode setting: INT4 g64 with an INT4 lm_head,
        # QKV / O / down / lm_head on v2 blocks (decoder.rs:361-390)
        "qwen64": (synth.QWEN_0_5B, 4, 4, 2048, 0x7B + 4),
    }[name]
    gs = 64 if name == "qwen64" else 32
    max_seq = kvlen + max(steps, 8)   # room for the 5-position verify at any step count
    w = synth.decoder_weights_torch(cfg, seed, wk, lk, gs)
    dec = decoder_from_weights(w, cfg, group_size=gs, max_seq_len=max_seq)
    del w
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 1)
    hkv, hd = cfg["num_kv_heads"], cfg["head_dim"]
    ks, vs = [], []
    for _ in range(cfg["num_layers"]):
        ks.append(torch.randn((hkv, kvlen, hd), device="cuda", generator=g))
        vs.append(torch.randn((hkv, kvlen, hd), device="cuda", generator=g))
    dec.copy_kv_cache_from_tensors(ks, vs, kvlen)
    del ks, vs
    torch.cuda.empty_cache()
    first = seed % cfg["vocab"]
    dec.time_greedy(first, kvlen, min(8, steps))          # warm-up (same positions)
    ms = dec.time_greedy(first, kvlen, steps)
    pre = prefill_run(dec, cfg, prefill_tokens) if prefill_tokens and wk == 4 else None
    sampled = sampled_run(dec, first, kvlen, steps) if name in ("llama4", "qwen64") else None
    verify = verify_run(dec, cfg, kvlen) if name == "llama4" else None
    dec.close()
    torch.cuda.empty_cache()
    byts = sum(synth.decode_bytes_per_token(cfg, kvlen + i, wk, lk, gs, v2=name == "qwen64")
               for i in range(steps)) / steps
    sec = ms / 1e3 / steps
    out = {"tok_s": round(1.0 / sec, 2), "ms_per_token": round(ms / steps, 4),
           "bytes_per_token": int(byts), "kv_len": kvlen,
           "roofline_frac": round(byts / sec / 1e9 / HBM_PEAK_GBS, 4),
           "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / byts, 1)}
    if pre:
        out["prefill"] = pre
    if sampled:
        out["sampled"] = sampled
    if verify:
        out["verify"] = verify
    return out


def verify_run(dec, cfg, kvlen, k=5):
    """verify_tokens of k draft positions as one batched forward against k
    single steps with logits (the reference's loop), wall clock of the C calls
    incl. the logits read back into host arrays (Python list conversion, which
    the reference's API also pays, excluded from both)."""
    toks = [int(t) for t in np.random.default_rng(3).integers(0, cfg["vocab"], k)]
    dec._verify(kvlen, toks)                             # warm-up
    t0 = time.perf_counter()
    dec._verify(kvlen, toks)
    batched = time.perf_counter() - t0
    t0 = time.perf_counter()
    for i, t in enumerate(toks):
        dec._step(t, kvlen + i, True)
    stepped = time.perf_counter() - t0
    return {"positions": k, "batched_ms": round(batched * 1e3, 3),
            "stepped_ms": round(stepped * 1e3, 3)}


def sampled_run(dec, first, kvlen, steps):
    """generate_loop with temperature 0.7, top_k 40, top_p 0.9 and repetition
    penalty 1.1 over the same positions (device sampler in the step graph), wall
    clock of the whole call."""
    args = dict(temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.1)
    dec.set_seed(1)
    dec.generate_loop(first, kvlen, min(8, steps), **args)          # warm-up, captures
    times = []
    for _ in range(2):
        dec.set_seed(1)
        t0 = time.perf_counter()
        toks, _ = dec.generate_loop(first, kvlen, steps, **args)
        times.append(time.perf_counter() - t0)
    sec = min(times) / steps
    return {"tok_s": round(1.0 / sec, 2), "ms_per_token": round(sec * 1e3, 4),
            "params": args, "tokens": steps}


def prefill_run(dec, cfg, n):
    """Batched prompt prefill of n tokens from an empty cache (wall clock of the
    whole call: token upload, every layer's kernels, lm_head, logits download)."""
    from torchburn_amd import synth
    g = np.random.default_rng(7)
    prompt = [int(t) for t in g.integers(0, cfg["vocab"], n)]
    dec.reset_kv_cache()
    dec.prefill_tokens(prompt, 0)                      # warm-up, allocates the batch buffers
    times = []
    for _ in range(3):
        dec.reset_kv_cache()
        t0 = time.perf_counter()
        dec.prefill_tokens(prompt, 0)
        times.append(time.perf_counter() - t0)
    sec = min(times)
    fl = synth.prefill_flops(cfg, n)
    return {"tokens": n, "ms": round(sec * 1e3, 3), "tok_s": round(n / sec, 1),
            "tflops": round(fl / sec / 1e12, 2), "flops": fl,
            "mfma_fp32_frac": round(fl / sec / 1e12 / MFMA_F32_PEAK, 4),
            "kernel": "k_w4_lgemm (f16 MFMA on exact limbs of x) for the projections; "
                      "mfma_fp32_frac is the f32-contraction rate over the FP32-MFMA peak"}


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU sharding is design-only",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import torch
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.calib_copy_mib:
        n = args.calib_copy_mib << 20
        a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"calib_copy_bytes": n, "copies": 5}))
        return

    t_start = time.perf_counter()
    r = mlp_section(torch, args, dev)
    gbs = r["step_bytes"] / (r["ms"] * 1e-3) / 1e9
    gu_gbs = r["gu_bytes"] / (r["gu_us"] * 1e-6) / 1e9
    batched = batched_section(torch, args, dev) if args.batched != "none" else {}
    mlp_batches = mlp_batch_section(torch, args, dev) if args.mlp_batches != "none" else {}
    cfg1 = None if args.no_config1 else config1_line(torch, dev)
    decode = {}
    if args.decode != "none":
        for name in args.decode.split(","):
            decode[name] = decode_run(torch, name.strip(), args.decode_steps,
                                      args.prefill_tokens if name.strip() == "llama4" else 0)
    if not args.no_cpu and args.cpu_decode != "none":
        for name in args.cpu_decode.split(","):
            if name in decode:
                decode[name]["cpu_baseline"] = cpu_decode(name)
    line = {
        "metric": "INT4 GEMV HBM GB/s (% of 8 TB/s); decode tokens/sec at 8B shape, 1 GPU",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "n_gpus": 1, "steps": r["steps"], "warmup": args.warmup,
        "ms_per_step": round(r["ms"], 5),
        "ms_per_step_spread": r["spread"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int4 weights, f32 activations, f32 accumulate",
        "data": "synthetic (seeded random weights and activations)",
        "config": {"workload": f"llama3-8b int4-g32 SwiGLU MLP step (gate/up + down + residual), "
                               f"M={args.m}", "m": args.m, "hidden": 4096,
                   "intermediate": 14336, "group_size": 32, "weight_copies_rotated": args.copies,
                   "step_bytes": r["step_bytes"], "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "kernel": "k_w4_gemv (gate/up pair, silu*up epilogue)",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                     "traffic": pmc_traffic() if args.m == 1 else None,
                     "traffic_source": "rocprofv3 --pmc FETCH_SIZE x2.0 + WRITE_SIZE x1.0 "
                                       "(copy-kernel calibration), "
                                       "profiles/k_w4_gemv_swiglu_llama8b_mlp_m1_pmc.md",
                     "avg_us": round(r["gu_us"], 3), "bytes_per_launch": r["gu_bytes"],
                     "down_kernel_avg_us": round(r["dn_us"], 3),
                     "down_kernel_gbs": round(r["dn_bytes"] / (r["dn_us"] * 1e-6) / 1e9, 1),
                     # fastest plain read of each kernel's weight + scale bytes
                     # (tb_read_probe over the same rotation of cold copies)
                     "read_ceiling": r["ceiling"],
                     "frac_of_read_ceiling": round(
                         gu_gbs / r["ceiling"]["gate_up"]["gbs"], 4)},
        "decode": decode,
        "batched_mfma": batched,
        "mlp_batches": mlp_batches,
        "config1": cfg1,
        "cpu_baseline": r["cpu"],
        "parity_max_rel": r["max_rel"],
        "wall_s": round(time.perf_counter() - t_start, 1),
    }
    if "llama4" in decode:
        line["decode_tok_s"] = decode["llama4"]["tok_s"]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

"""Benchmark of the gfx950 INT4 decode hot path.

Default workload: the Llama-3-8B-shape INT4 (group 32)
SwiGLU MLP at batch M = 1 -- gate/up [14336, 4096] fused with silu*up, then down
[4096, 14336] with the residual add -- on one MI355X.  One "step" is one pass of
that MLP over one synthetic activation row; inputs are resident in HBM before
the timed region.  Four distinct weight copies (4 x 110 MB) are rotated so the
256 MB Infinity Cache cannot serve the weights.

Prints one JSON line (rank 0): metric/value = whole-step algorithmic bytes per
second (GB/s), plus the roofline of the dominant kernel (the fused gate/up
GEMV, timed with HIP events on its own stream) and the CPU-oracle baseline
timed on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
ROOT = os.path.dirname(os.path.abspath(__file__))


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--m", type=int, default=1, help="activation rows (config 2: 1, 4, 8)")
    ap.add_argument("--copies", type=int, default=4, help="weight copies rotated (> 256 MB)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (FETCH_SIZE / "
                         "WRITE_SIZE calibration for rocprofv3 --pmc), then exit")
    return ap.parse_args()


def cpu_info():
    model, flags = "", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and not model:
                    model = line.split(":", 1)[1].strip()
                if line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return model, sorted(f for f in flags if f in ("avx2", "fma", "avx512f", "avx512bw",
                                                    "avx512_vnni"))


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU sharding is "
                                   "design-only (see DESIGN.md)", "n_gpus": args.gpus}))
        sys.exit(2)

    import torch
    import torchburn_amd as tb
    from torchburn_amd import synth

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
    M, K, I, GS = args.m, 4096, 14336, 32

    # Weights: `copies` independent sets generated on the device.
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x7B + 2)

    def int4(n, k):
        w = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=dev, generator=gen)
        s = torch.randn((n, k // GS), device=dev, generator=gen).mul_(0.02).abs_().add_(1e-3)
        return w, s

    sets = []
    for _ in range(args.copies):
        gw, gs = int4(I, K)
        uw, us = int4(I, K)
        dw, ds = int4(K, I)
        sets.append((gw, gs, uw, us, dw, ds))
    x = torch.randn((M, K), device=dev, generator=gen)
    r = torch.randn((M, K), device=dev, generator=gen)
    out = torch.empty((M, K), device=dev)
    h = torch.empty((M, I), device=dev)
    torch.cuda.synchronize()

    from torchburn_amd import _lib
    st = torch.cuda.current_stream(dev).cuda_stream
    P = lambda t: t.data_ptr()

    def gateup(ws):
        gw, gs, uw, us, _, _ = ws
        _lib.call("tb_swiglu_w4a32", P(x), P(gw), P(gs), None, P(uw), P(us), None, P(h),
                  M, K, I, GS, st)

    def down(ws):
        _, _, _, _, dw, ds = ws
        _lib.call("tb_w4a32_grouped_linear_residual", P(h), P(dw), P(ds), None, P(r), P(out),
                  M, K, I, GS, st)

    def step(i):
        ws = sets[i % len(sets)]
        gateup(ws)
        down(ws)

    w_bytes = 3 * (I * K // 2 + 4 * I * (K // GS))
    act_bytes = 4 * (M * K + 2 * M * I + 2 * M * K)  # x; h written+read; r; out
    step_bytes = w_bytes + act_bytes

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(args.steps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    gbs = step_bytes / (ms * 1e-3) / 1e9

    # Dominant kernel: the fused gate/up GEMV, timed alone over the same rotation.
    gu_bytes = 2 * (I * K // 2 + 4 * I * (K // GS)) + 4 * M * K + 4 * M * I
    for i in range(args.warmup):
        gateup(sets[i % len(sets)])
    e0.record()
    for i in range(args.steps):
        gateup(sets[i % len(sets)])
    e1.record()
    torch.cuda.synchronize()
    gu_us = e0.elapsed_time(e1) * 1e3 / args.steps
    gu_gbs = gu_bytes / (gu_us * 1e-6) / 1e9

    # Correctness guard on the measured data (oracle, CPU): one row of set 0.
    from oracle import oracle as O
    ws = [t.cpu().numpy() for t in sets[0]]
    xs, rs = x.cpu().numpy(), r.cpu().numpy()
    step(0)
    torch.cuda.synchronize()
    ref = O.swiglu_mlp_w4(xs, ws[0], ws[1], ws[2], ws[3], ws[4], ws[5], group_size=GS) + rs
    got = out.cpu().numpy()
    max_rel = float(np.abs(got - ref).max() / np.abs(ref).max())

    cpu = None
    if not args.no_cpu:
        n, t_start = 0, time.perf_counter()
        while True:
            O.swiglu_mlp_w4(xs, ws[0], ws[1], ws[2], ws[3], ws[4], ws[5], group_size=GS)
            n += 1
            el = time.perf_counter() - t_start
            if el > args.cpu_seconds:
                break
        model, flags = cpu_info()
        cpu = {"value": round(step_bytes * n / el / 1e9, 3), "unit": "GB/s",
               "cores": O.num_threads(), "kind": "port",
               "sample": f"{n} MLP passes (M={M}) of the C oracle in {el:.1f} s on {model} "
                         f"[{' '.join(flags)}]",
               "ms_per_step": round(el / n * 1e3, 3)}

    line = {
        "metric": "INT4 GEMV HBM GB/s (Llama-3-8B SwiGLU MLP, group 32)",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int4-w/f32-a (fp32 accumulate)", "data": "synthetic",
        "config": {"workload": f"llama3-8b int4-g32 swiglu mlp (gate/up+down+residual), M={M}",
                   "m": M, "hidden": K, "intermediate": I, "group_size": GS,
                   "weight_copies_rotated": args.copies, "step_bytes": step_bytes,
                   "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "kernel": "k_w4_gemv<dual swiglu>",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "avg_us": round(gu_us, 3), "bytes_per_launch": gu_bytes},
        "cpu_baseline": cpu,
        "parity_max_rel": max_rel,
        "wall_s": round(wall, 3),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

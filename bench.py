#!/usr/bin/env python3
"""Benchmark of the hot path on one MI355X.

Workload: single-token Q4_K GEMV at Llama-3-8B
shapes -- per layer 4096x4096 (x: 4096), 14336x4096 (x: 4096) and 4096x14336
(x: 14336) -- over 32 layers of distinct weights (2.42 GB, ten times the
256 MB Infinity Cache, so every weight byte comes from HBM).  Weights are
f32 ~ N(0, 0.02) quantised to Q4_K on the device; activations ~ N(0, 1).
One step = the 96 GEMVs of one decode token, each with its activation
quantisation, replayed from a HIP graph.  Inputs are resident in HBM.

value = algorithmic bytes per step / step time (GB/s), the bytes being
144*rows*cols/256 + 4*cols + 4*rows per GEMV.  roofline = the GEMV kernel
alone (graph of the 96 kernel launches on pre-quantised activations), timed
with HIP events on the stream it runs on.  cpu_baseline = the C oracle's Q4_K
GEMV on the host's cores over layer 0's three matrices.

Prints one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
LLAMA = [(4096, 4096), (14336, 4096), (4096, 14336)]
QWEN_FFN = [(4864, 896), (4864, 896), (896, 4864)]


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def q4k_bytes(rows, cols):
    return 144 * rows * cols // 256 + 4 * cols + 4 * rows


def q8_bytes(rows, cols):
    return rows * cols + 4 * rows * cols // 32 + 4 * cols + 4 * rows


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bound on the CPU-baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the secondary (q8, attention) figures")
    return ap.parse_args()


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor() or "unknown"


class Graph:
    """A HIP graph of library launches captured on a private stream."""

    def __init__(self, torch, ctx, stream, fn):
        self.torch, self.stream = torch, stream
        fn()  # eager once: allocations happen here, not under capture
        torch.cuda.synchronize()
        self.g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.g, stream=stream):
            fn()
        torch.cuda.synchronize()

    def time(self, reps: int, warmup: int) -> float:
        """Seconds per replay, HIP events on the graph's stream."""
        torch = self.torch
        with torch.cuda.stream(self.stream):
            for _ in range(warmup):
                self.g.replay()
            torch.cuda.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(self.stream)
            for _ in range(reps):
                self.g.replay()
            e1.record(self.stream)
            e1.synchronize()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3 / reps


def main() -> int:
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU; --gpus N > 1 is not supported "
              "(the sharding design is described in DESIGN.md)", file=sys.stderr)
        return 2

    import torch

    import kvad_amd as K

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ctx = K.Context(0)
    stream = torch.cuda.Stream()
    ctx.set_stream(stream.cuda_stream)
    ctx.reserve(64 << 20)
    gen = torch.Generator(device=dev)
    gen.manual_seed(20251201)

    # ---- weights: Q4_K quantised on the device from f32 ~ N(0, 0.02) ------
    t0 = time.time()
    layers = []
    with torch.cuda.stream(stream):
        for l in range(args.layers):
            ws = []
            for rows, cols in LLAMA:
                f = torch.randn(rows, cols, device=dev, generator=gen) * 0.02
                ws.append(K.Weight.quantize_dev(ctx, rows, cols, f.data_ptr(), K.Q4K))
                del f
            x4 = torch.randn(4096, device=dev, generator=gen)
            x14 = torch.randn(14336, device=dev, generator=gen)
            ys = [torch.empty(r, device=dev) for r, _ in LLAMA]
            layers.append((ws, [x4, x4, x14], ys))
    ctx.synchronize()
    torch.cuda.synchronize()
    log(f"quantised {args.layers} layers of Q4_K weights in {time.time() - t0:.1f}s")
    step_bytes = sum(q4k_bytes(r, c) for r, c in LLAMA) * args.layers
    weight_bytes = sum(w.bytes for ws, _, _ in layers for w in ws)

    def step():
        for ws, xs, ys in layers:
            for w, x, y in zip(ws, xs, ys):
                w.matvec_bt_dev(x.data_ptr(), y.data_ptr())

    g_step = Graph(torch, ctx, stream, step)
    sec = g_step.time(args.steps, args.warmup)
    log(f"step: {sec * 1e3:.3f} ms, {step_bytes / sec / 1e9:.1f} GB/s")

    # ---- the GEMV kernel alone, on pre-quantised activations --------------
    acts = {}
    with torch.cuda.stream(stream):
        for l, (ws, xs, ys) in enumerate(layers):
            for i, x in enumerate(xs):
                n = x.numel()
                qs = torch.empty(n, dtype=torch.int8, device=dev)
                sc = torch.empty(n // 32, device=dev)
                su = torch.empty(n // 32, dtype=torch.int32, device=dev)
                K.qact_dev(ctx, x.data_ptr(), 1, n, qs.data_ptr(), sc.data_ptr(), su.data_ptr())
                acts[(l, i)] = (qs, sc, su)
    torch.cuda.synchronize()

    def kernels(shape_idx=None):
        def run():
            for l, (ws, xs, ys) in enumerate(layers):
                for i, (w, y) in enumerate(zip(ws, ys)):
                    if shape_idx is not None and i != shape_idx:
                        continue
                    qs, sc, su = acts[(l, i)]
                    w.matvec_q_dev(qs.data_ptr(), sc.data_ptr(), su.data_ptr(), y.data_ptr())
        return run

    g_k = Graph(torch, ctx, stream, kernels())
    ksec = g_k.time(args.steps, args.warmup)
    launches = 3 * args.layers
    avg_launch = ksec / launches
    achieved = step_bytes / ksec / 1e9
    log(f"gemv kernels: {avg_launch * 1e6:.2f} us/launch avg, {achieved:.1f} GB/s")
    per_shape = {}
    for i, (rows, cols) in enumerate(LLAMA):
        g = Graph(torch, ctx, stream, kernels(i))
        s = g.time(args.steps, args.warmup) / args.layers
        per_shape[f"{rows}x{cols}"] = {"us": round(s * 1e6, 3), "GBps": round(q4k_bytes(rows, cols) / s / 1e9, 1)}
        del g
    log(f"per shape: {per_shape}")

    extra = {"q4k_gemv_per_shape": per_shape, "weight_bytes_resident": weight_bytes}
    if not args.no_extra:
        extra.update(secondary(torch, K, ctx, stream, dev, gen, args))

    # ---- CPU baseline: the oracle on the host's cores ---------------------
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(layers, args.cpu_seconds)

    result = {
        "metric": "Q4_K GEMV achieved GB/s at Llama-3-8B shapes (single-token decode)",
        "value": round(step_bytes / sec / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights x int8 activations, i32 block dots, f32 accumulate",
        "data": "synthetic: W ~ N(0,0.02) quantised to Q4_K on device, x ~ N(0,1)",
        "config": {"workload": "q4k-gemv-llama3-8b", "layers": args.layers,
                   "shapes": ["4096x4096", "14336x4096", "4096x14336"], "gemvs_per_step": launches,
                   "bytes_per_step": step_bytes, "launch": "hip graph"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": "gemv_kernel<Q4K>", "avg_launch_us": round(avg_launch * 1e6, 3),
                     "bytes_per_launch": step_bytes // launches},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(result), flush=True)
    ctx.set_stream(None)
    return 0


def secondary(torch, K, ctx, stream, dev, gen, args):
    """BASELINE configs[0] (Q8 GEMV at Qwen2.5-0.5B FFN shapes, 24 layers) and
    configs[3] (decode attention, Qwen geometry) as extra figures."""
    out = {}
    qlayers = []
    with torch.cuda.stream(stream):
        for l in range(24):
            ws = []
            for rows, cols in QWEN_FFN:
                f = torch.randn(rows, cols, device=dev, generator=gen) * 0.02
                ws.append(K.Weight.quantize_dev(ctx, rows, cols, f.data_ptr(), K.Q8))
            x = torch.randn(896, device=dev, generator=gen)
            h = torch.randn(4864, device=dev, generator=gen)
            ys = [torch.empty(r, device=dev) for r, _ in QWEN_FFN]
            qlayers.append((ws, [x, x, h], ys))
    torch.cuda.synchronize()
    qbytes = 24 * sum(q8_bytes(r, c) for r, c in QWEN_FFN)

    def step():
        for ws, xs, ys in qlayers:
            for w, x, y in zip(ws, xs, ys):
                w.matvec_bt_dev(x.data_ptr(), y.data_ptr())

    g = Graph(torch, ctx, stream, step)
    s = g.time(args.steps, args.warmup)
    out["q8_gemv_qwen05b_ffn"] = {"GBps": round(qbytes / s / 1e9, 1), "us_per_gemv": round(s / 72 * 1e6, 3),
                                  "bytes_per_step": qbytes}
    log(f"q8 qwen ffn: {out['q8_gemv_qwen05b_ffn']}")
    del g

    spec = K.Spec(14, 2, 64)
    att = {}
    for L in (1024, 8192, 32768):
        nl = 24
        kv = torch.randn(nl, 2, L, 128, device=dev, generator=gen)
        q = torch.randn(14 * 64, device=dev, generator=gen)
        o = torch.empty(14 * 64, device=dev)

        def run():
            for l in range(nl):
                K.attend_dev(ctx, spec, q.data_ptr(), kv[l, 0].data_ptr(), kv[l, 1].data_ptr(), L, o.data_ptr())

        g = Graph(torch, ctx, stream, run)
        s = g.time(max(5, args.steps // 5), 2) / nl
        b = 4 * L * 256 + 8 * 14 * 64
        att[str(L)] = {"us_per_layer": round(s * 1e6, 2), "GBps": round(b / s / 1e9, 1)}
        del g, kv
    out["attend_qwen05b"] = att
    log(f"attend: {att}")
    return out


def cpu_baseline(layers, budget_s: float):
    import numpy as np

    import oracle as O

    ws = layers[0][0]
    xs = [x.cpu().numpy() for x in layers[0][1]]
    parts = [w.parts()[1] for w in ws]
    threads = O.threads()

    def one():
        for (rows, cols), b, x in zip(LLAMA, parts, xs):
            O.matvec_q4k(b, rows, cols, x)

    t = time.perf_counter()
    one()
    first = time.perf_counter() - t
    rounds, best = 0, float("inf")
    deadline = time.perf_counter() + budget_s
    while rounds < 5 and time.perf_counter() < deadline:
        t = time.perf_counter()
        one()
        best = min(best, time.perf_counter() - t)
        rounds += 1
    nbytes = sum(q4k_bytes(r, c) for r, c in LLAMA)
    # parity spot check of what was timed against the device result
    ys = [y.cpu().numpy() for y in layers[0][2]]
    y0 = O.matvec_q4k(parts[0], 4096, 4096, xs[0])
    agree = float(np.max(np.abs(y0 - ys[0])) / max(np.max(np.abs(y0)), 1e-30))
    log(f"cpu oracle: {best * 1e3:.1f} ms per 3 GEMVs on {threads} threads ({nbytes / best / 1e9:.1f} GB/s); "
        f"first {first:.2f}s; device-vs-oracle rel err {agree:.2e}")
    return {"value": round(nbytes / best / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"oracle matvec_q4k over layer 0's three matrices ({nbytes / 1e6:.1f} MB), best of {rounds}",
            "cpu": cpu_model(), "rel_err_vs_device": agree}


if __name__ == "__main__":
    sys.exit(main())

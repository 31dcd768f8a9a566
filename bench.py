#!/usr/bin/env python3
"""Benchmark of the hot path on one MI355X.

Workload: single-token Q4_K GEMV at Llama-3-8B
shapes, as one decode token issues them: per layer the q/k/v projections
(4096 + 1024 + 1024 rows x 4096, one matvec_many launch, as they share
their input), o (4096x4096), gate+up (2 x 14336x4096, one matvec_many
launch) and down (4096x14336) -- 32 layers of distinct weights (3.9 GB,
fifteen times the 256 MB Infinity Cache, so every weight byte comes from
HBM).  Weights are f32 ~ N(0, 0.02) quantised to Q4_K on the device;
activations ~ N(0, 1) (synthetic, independent per projection).  One step =
the 128 GEMV launches of one token, each with its activation quantisation,
replayed from a HIP graph.  Inputs are resident in HBM.

value = algorithmic bytes per step / step time (GB/s), the bytes being
144*rows*cols/256 + 4*cols + 4*rows per GEMV.  roofline: every launch of the
step is the GEMV kernel (it quantises its own input), so its average launch
duration is the step time over the 128 launches, timed with HIP events on
the stream they run on.  cpu_baseline = the C oracle's Q4_K GEMV on the
host's cores over layer 0's matrices.

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

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
LLAMA = [(4096, 4096), (14336, 4096), (4096, 14336)]
LLAMA_LAYER = {"q": (4096, 4096), "k": (1024, 4096), "v": (1024, 4096), "o": (4096, 4096),
               "gate": (14336, 4096), "up": (14336, 4096), "down": (4096, 14336)}
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
    ap.add_argument("--cpu-column-seconds", type=float, default=0.6,
                    help="bound on each secondary figure's CPU column (the oracle beside it)")
    ap.add_argument("--no-extra", action="store_true", help="skip the secondary (q8, attention) figures")
    ap.add_argument("--only", choices=SECTIONS, default=None,
                    help="run one secondary workload alone (for per-kernel rocprofv3 summaries) and print its figures")
    ap.add_argument("--counters", type=int, default=0, metavar="MIB",
                    help="only run a MIB-sized copy and two eager steps of the GEMV kernels (for rocprofv3 --pmc)")
    ap.add_argument("--gemm-counters", action="store_true",
                    help="only run three eager q8 prefill GEMMs per shape (for rocprofv3 --pmc)")
    ap.add_argument("--kernel-counters", choices=("moe_decode", "moe_prefill", "mla", "attend"), default=None,
                    help="only run a few eager launches of one secondary workload (for rocprofv3 --pmc)")
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

    def time(self, reps: int, warmup: int, settle: float = 0.0) -> float:
        """Seconds per replay, HIP events on the graph's stream.  With settle
        > 0 the graph is also replayed for that many seconds first: the
        matrix-core clocks rise over the first second or so of sustained
        load (a compute-bound GEMM measured 468, 394, 381 us on one box as
        it warmed), so compute-bound figures are taken once they hold."""
        torch = self.torch
        with torch.cuda.stream(self.stream):
            for _ in range(warmup):
                self.g.replay()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            while time.perf_counter() - t0 < settle:
                for _ in range(4):
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
              "(value is one GPU's throughput on its share of the path)", file=sys.stderr)
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

    if args.gemm_counters:
        # a workload for rocprofv3 --pmc: the q8 prefill GEMM at the two
        # prefill configurations and at 32 rows of mlp.down (k-stages split)
        shapes = ((512, 896, 4864), (2048, 4096, 14336), (32, 4864, 896))
        for (m, k, n) in shapes:
            f = torch.randn(n, k, device=dev, generator=gen) * 0.02
            xs = torch.randn(m, k, device=dev, generator=gen)
            y = torch.empty(m, n, device=dev)
            with torch.cuda.stream(stream):
                w = K.Weight.quantize_dev(ctx, n, k, f.data_ptr(), K.Q8)
                for _ in range(3):
                    w.matmul_bt_dev(xs.data_ptr(), m, y.data_ptr())
            torch.cuda.synchronize()
            del w, f, xs, y
        print(json.dumps({"gemm_counters_run": {"shapes_mkn": shapes, "calls_each": 3}}), flush=True)
        ctx.set_stream(None)
        return 0

    if args.kernel_counters:
        counter_workload(torch, K, ctx, stream, dev, gen, args.kernel_counters)
        ctx.set_stream(None)
        return 0

    if args.only:
        rig = None if args.no_cpu else CpuRig(args.cpu_column_seconds)
        res = secondary(torch, K, ctx, stream, dev, gen, args, only=args.only, rig=rig)
        print(json.dumps({"section": args.only, "n_gpus": 1, "data": "synthetic", "extra": res}), flush=True)
        ctx.set_stream(None)
        return 0

    # ---- weights: Q4_K quantised on the device from f32 ~ N(0, 0.02) ------
    t0 = time.time()
    layers = []
    with torch.cuda.stream(stream):
        for l in range(args.layers):
            L = {}
            for name, (rows, cols) in LLAMA_LAYER.items():
                f = torch.randn(rows, cols, device=dev, generator=gen) * 0.02
                L[name] = K.Weight.quantize_dev(ctx, rows, cols, f.data_ptr(), K.Q4K)
                L["y_" + name] = torch.empty(rows, device=dev)
                del f
            for name, n in (("x", 4096), ("a", 4096), ("h", 4096), ("m", 14336)):
                L[name] = torch.randn(n, device=dev, generator=gen)
            layers.append(L)
    ctx.synchronize()
    torch.cuda.synchronize()
    log(f"quantised {args.layers} layers of Q4_K weights in {time.time() - t0:.1f}s")
    step_bytes = args.layers * sum(q4k_bytes(r, c) for r, c in LLAMA_LAYER.values())
    weight_bytes = sum(L[n].bytes for L in layers for n in LLAMA_LAYER)
    launches = 4 * args.layers

    def many(ws, xs, ys):
        n = len(ws)
        arr = lambda vals: (K.C.c_void_p * n)(*vals)
        rc = K.lib.kh_matvec_many_dev(ctx.h, n, arr([w.h.value for w in ws]), arr(xs), arr(ys))
        assert rc == 0, K.lib.kh_last_error()

    def step():
        for L in layers:
            many([L["q"], L["k"], L["v"]], [L["x"].data_ptr()] * 3,
                 [L["y_q"].data_ptr(), L["y_k"].data_ptr(), L["y_v"].data_ptr()])
            L["o"].matvec_bt_dev(L["a"].data_ptr(), L["y_o"].data_ptr())
            many([L["gate"], L["up"]], [L["h"].data_ptr()] * 2, [L["y_gate"].data_ptr(), L["y_up"].data_ptr()])
            L["down"].matvec_bt_dev(L["m"].data_ptr(), L["y_down"].data_ptr())

    if args.counters:
        # a workload for rocprofv3 --pmc: a streaming kernel of known traffic
        # (dst = 2 * src over MIB MiB each way, far past the 256 MB cache: the
        # counters' calibration), then the GEMV kernels launched eagerly
        n = args.counters << 18  # MiB -> floats
        src = torch.ones(n, device=dev)
        dst = torch.empty(n, device=dev)
        torch.cuda.synchronize()
        for _ in range(3):
            torch.mul(src, 2.0, out=dst)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            for _ in range(2):
                step()
        torch.cuda.synchronize()
        print(json.dumps({"counters_run": {"calibration_bytes_each_way": 4 * n, "calibration_runs": 3, "gemv_steps": 2,
                                           "launches_per_step": launches, "bytes_per_step": step_bytes}}))
        return 0

    # every launch of the step is a GEMV kernel (each quantises its own
    # input), so the step's events time the kernel: avg launch = step / launches
    g_step = Graph(torch, ctx, stream, step)
    sec = g_step.time(args.steps, args.warmup)
    avg_launch = sec / launches
    achieved = step_bytes / sec / 1e9
    log(f"step: {sec * 1e3:.3f} ms, {achieved:.1f} GB/s, {avg_launch * 1e6:.2f} us per GEMV launch")

    # ---- the structure's ceiling: the same 128 launches reading the same
    # weight bytes with a plain streaming kernel (no activation, no
    # arithmetic), its launch shape swept; the GEMV's step over it -------------
    sink = torch.empty(4096, dtype=torch.int32, device=dev)
    wbytes_step = sum(L[n].bytes for L in layers for n in LLAMA_LAYER)

    def probe_step():
        for L in layers:
            K.stream_dev(ctx, [L["q"], L["k"], L["v"]], sink.data_ptr())
            K.stream_dev(ctx, [L["o"]], sink.data_ptr())
            K.stream_dev(ctx, [L["gate"], L["up"]], sink.data_ptr())
            K.stream_dev(ctx, [L["down"]], sink.data_ptr())

    # 32 waves per CU in three workgroup sizes (fewer measured slower), with
    # and without the non-temporal cache policy
    knobs = ("KVAD_STREAM_WG_PER_CU", "KVAD_STREAM_THREADS", "KVAD_STREAM_NT")
    best, sweep = None, {}
    for wg, thr in ((8, 256), (4, 512), (2, 1024)):
        for nt in (0, 1):
            for k, v in zip(knobs, (wg, thr, nt)):
                os.environ[k] = str(v)
            g = Graph(torch, ctx, stream, probe_step)
            s = g.time(max(5, args.steps // 4), 2)
            del g
            sweep[f"{wg}x{thr}{' nt' if nt else ''}"] = round(s * 1e3, 4)
            if best is None or s < best[0]:
                best = (s, wg, thr, nt)
    for k in knobs:
        os.environ.pop(k)
    ceiling = {"ms_per_step": round(best[0] * 1e3, 4), "weight_GBps": round(wbytes_step / best[0] / 1e9, 1),
               "launch": {"workgroups_per_cu": best[1], "threads_per_workgroup": best[2],
                          "non_temporal": bool(best[3])},
               "sweep_ms_per_step": sweep,
               "gemv_step_over_ceiling": round(sec / best[0], 3),
               "gemv_weight_GBps": round(wbytes_step / sec / 1e9, 1)}
    log(f"structure ceiling: {ceiling}")

    # ---- each config shape as its own launch ------------------------------
    per_shape = {}
    for name in ("o", "up", "down"):
        rows, cols = LLAMA_LAYER[name]

        def one():
            for L in layers:
                L[name].matvec_bt_dev(L["m" if name == "down" else "x"].data_ptr(), L["y_" + name].data_ptr())

        g = Graph(torch, ctx, stream, one)
        s = g.time(args.steps, args.warmup) / args.layers
        per_shape[f"{rows}x{cols}"] = {"us": round(s * 1e6, 3), "GBps": round(q4k_bytes(rows, cols) / s / 1e9, 1)}
        del g

        def probe_one():
            for L in layers:
                K.stream_dev(ctx, [L[name]], sink.data_ptr())

        for k, v in zip(knobs, best[1:]):
            os.environ[k] = str(int(v))
        g = Graph(torch, ctx, stream, probe_one)
        sp = g.time(args.steps, args.warmup) / args.layers
        del g
        for k in knobs:
            os.environ.pop(k)
        per_shape[f"{rows}x{cols}"]["ceiling_us"] = round(sp * 1e6, 3)
    log(f"per shape: {per_shape}")

    # the dequantising kernel (quant.rs:522-589) on the same step: one launch
    # per matrix, as the reference runs matvec_many's jobs one at a time under
    # KVAD_DEQUANT (quant.rs:629-633)
    def dq_step():
        for L in layers:
            for n, xin in (("q", "x"), ("k", "x"), ("v", "x"), ("o", "a"), ("gate", "h"), ("up", "h"), ("down", "m")):
                L[n].matvec_bt_dequant_dev(L[xin].data_ptr(), L["y_" + n].data_ptr())

    g = Graph(torch, ctx, stream, dq_step)
    s_dq = g.time(max(3, args.steps // 2), args.warmup)
    del g
    dequant_step = {"ms_per_step": round(s_dq * 1e3, 4), "GBps": round(step_bytes / s_dq / 1e9, 1),
                    "launches_per_step": 7 * args.layers}
    log(f"dequant q4k step: {dequant_step}")

    # ---- batched decode (forward_each, llama.rs:418-434): m tokens through
    # the same 32 layers, one matmul_bt per projection: one multi-token GEMV
    # launch streams the weights once, quantising the m rows in every
    # workgroup while 2/4/8 token slots x cols <= 12288, else after a
    # quantising launch of its own -------------------------------------------
    batched = {}
    xs_m = torch.randn(8 * 14336, device=dev, generator=gen)
    ys_m = torch.empty(8 * 14336, device=dev)
    for m in (2, 4, 8):
        def bstep(m=m):
            for L in layers:
                for name in LLAMA_LAYER:
                    L[name].matmul_bt_dev(xs_m.data_ptr(), m, ys_m.data_ptr())

        g = Graph(torch, ctx, stream, bstep)
        s = g.time(max(3, args.steps // 2), args.warmup)
        bb = args.layers * sum(144 * r * c // 256 + 4 * m * (r + c) for r, c in LLAMA_LAYER.values())
        batched[str(m)] = {"ms_per_step": round(s * 1e3, 4), "GBps": round(bb / s / 1e9, 1),
                           "token_rows_per_s": round(m / s, 1),
                           "launches_per_step": args.layers * sum(1 if (2 if m <= 2 else 4 if m <= 4 else 8) * c <= 12288
                                                                  else 2 for _, c in LLAMA_LAYER.values())}
        del g
    log(f"batched decode q4k: {batched}")

    extra = {"q4k_gemv_per_shape": per_shape, "weight_bytes_resident": weight_bytes,
             "q4k_step_structure_ceiling": ceiling,
             "q4k_dequant_step": dequant_step, "q4k_batched_decode_llama3_8b": batched}
    rig = None if args.no_cpu else CpuRig(args.cpu_column_seconds)
    if not args.no_extra:
        extra.update(secondary(torch, K, ctx, stream, dev, gen, args, rig=rig))

    # ---- CPU baseline: the oracle on the host's cores ---------------------
    cpu = None
    if rig is not None:
        cpu = cpu_baseline(layers, args.cpu_seconds, rig)

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
        "config": {"workload": "q4k-gemv-llama3-8b-decode", "layers": args.layers,
                   "per_layer": "qkv 6144x4096 (one launch), o 4096x4096, gate+up 28672x4096 (one launch), "
                                "down 4096x14336", "launches_per_step": launches,
                   "bytes_per_step": step_bytes, "launch": "hip graph"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": measured_traffic(),
                     "kernel": "gemv_kernel<Q4K,*>", "avg_launch_us": round(avg_launch * 1e6, 3),
                     "bytes_per_launch": step_bytes // launches},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(result), flush=True)
    ctx.set_stream(None)
    return 0


def counter_workload(torch, K, ctx, stream, dev, gen, name, reps=3):
    """Eager launches of one secondary figure's kernels, for rocprofv3 --pmc
    passes (graph replays hide per-dispatch counters): the DeepSeek-V2-Lite
    MoE decode layer (4 distinct layers, one token) or prefill (one layer,
    512 tokens), latent attention at
    L = 32768 (4 layers of distinct caches), or GQA attention at Qwen2.5-0.5B
    geometry and L = 32768 (8 layers)."""
    with torch.cuda.stream(stream):
        if name in ("moe_decode", "moe_prefill"):
            hidden, inter, n_exp, k, sh = 2048, 1408, 64, 6, 2816
            n_layers, M = (4, 1) if name == "moe_decode" else (1, 512)

            def q8(rows, cols, sd=0.02):
                f = torch.randn(rows, cols, device=dev, generator=gen) * sd
                return K.Weight.quantize_dev(ctx, rows, cols, f.data_ptr(), K.Q8)

            layers = []
            for _ in range(n_layers):
                m = K.Moe(ctx, n_exp, k, hidden, inter)
                m.set_router(q8(n_exp, hidden, 0.5))
                for x in range(n_exp):
                    m.set_expert(x, q8(inter, hidden), q8(inter, hidden), q8(hidden, inter))
                m.set_shared(q8(sh, hidden), q8(sh, hidden), q8(hidden, sh))
                layers.append((m, torch.randn(M, hidden, device=dev, generator=gen),
                               torch.empty(M, hidden, device=dev)))
            torch.cuda.synchronize()
            for _ in range(reps):
                for m, x, y in layers:
                    m.run_dev(x.data_ptr(), M, y.data_ptr())
        elif name == "mla":
            L, H = 32768, 16
            c = torch.randn(4, L, 512, device=dev, generator=gen)
            pe = torch.randn(4, L, 64, device=dev, generator=gen)
            ql = torch.randn(H * 512, device=dev, generator=gen)
            qp = torch.randn(H * 64, device=dev, generator=gen)
            o = torch.empty(H * 512, device=dev)
            torch.cuda.synchronize()
            for _ in range(reps):
                for l in range(4):
                    K.mla_attend_dev(ctx, H, ql.data_ptr(), qp.data_ptr(), c[l].data_ptr(), pe[l].data_ptr(), L,
                                     1.0 / 192 ** 0.5, o.data_ptr())
        else:
            L, spec = 32768, K.Spec(14, 2, 64)
            kv = torch.randn(8, 2, L, 128, device=dev, generator=gen)
            q = torch.randn(14 * 64, device=dev, generator=gen)
            o = torch.empty(14 * 64, device=dev)
            torch.cuda.synchronize()
            for _ in range(reps):
                for l in range(8):
                    K.attend_dev(ctx, spec, q.data_ptr(), kv[l, 0].data_ptr(), kv[l, 1].data_ptr(), L, o.data_ptr())
    torch.cuda.synchronize()
    print(json.dumps({"kernel_counters_run": name, "reps": reps}), flush=True)


TRAFFIC = ROOT / "profiles" / "gemv_q4k_llama3_8b_traffic.json"


def measured_traffic():
    """HBM bytes per GEMV launch of this workload, from the rocprofv3 --pmc
    passes recorded in profiles/ (FETCH_SIZE + WRITE_SIZE per dispatch, each
    scaled by what the counter reads for a plain copy of known size); null
    until those passes exist."""
    try:
        return json.loads(TRAFFIC.read_text())["bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        return None


SECTIONS = ("q8", "prefill", "moe", "decode", "attend", "mla", "qcache", "session_prefill")


def secondary(torch, K, ctx, stream, dev, gen, args, only=None, rig=None):
    """The other configs as extra figures: BASELINE configs[0] (Q8 GEMV at
    Qwen2.5-0.5B shapes), [2] (prefill GEMM), [3] (decode attention), [4]
    (MoE) and the Qwen2.5-0.5B q8 decode session.  `only` picks one.  With a
    CpuRig each figure carries a "cpu" entry: the oracle on the host's cores,
    timed in the same run."""
    out = {}
    want = lambda name: only is None or only == name
    if want("q8"):
        out.update(q8_qwen(torch, K, ctx, stream, dev, gen, args, rig))
    if want("prefill"):
        out["prefill_gemm"] = prefill(torch, K, ctx, stream, dev, gen, args, rig)
    if want("moe"):
        out["moe_deepseek_v2_lite"] = moe(torch, K, ctx, stream, dev, gen, args, rig=rig)
    if want("decode"):
        out["qwen05b_q8_decode"] = decode(torch, K, ctx, stream, dev, gen, args, rig=rig)
    if only == "session_prefill":  # the prompt passes alone (inside "decode" otherwise)
        m, host = qwen05b_session(torch, K, ctx, stream, dev, gen)
        out["qwen05b_q8_prefill"] = prefill_session(m, rig=rig, host=host)
        m.free()
    if want("attend"):
        out["attend_qwen05b"] = attend(torch, K, ctx, stream, dev, gen, args, rig)
    if want("mla"):
        out["mla_deepseek_v2_lite"] = mla(torch, K, ctx, stream, dev, gen, args, rig)
    if want("qcache"):
        out["qcache_upload"] = qcache_upload(K, ctx)
    return out


def mla_cpu(rig, H, L):
    """The oracle's absorbed latent attention (deepseek.rs:553-591, parallel
    over heads) on the host, over layers of distinct latent caches."""
    O = rig.O
    per = 4 * L * 576
    nl = rig.layers_past_llc(per, hi=8)
    rng = np.random.default_rng(L)
    c = rng.standard_normal((nl, L, 512), dtype=np.float32)
    pe = rng.standard_normal((nl, L, 64), dtype=np.float32)
    ql = rng.standard_normal(H * 512, dtype=np.float32)
    qp = rng.standard_normal(H * 64, dtype=np.float32)
    b = per + 4 * H * (512 + 64 + 512)

    def make(lib, nt):
        def run():
            for l in range(nl):
                O.mla_attend(H, 512, 64, ql, qp, c[l], pe[l], L, 1.0 / 192 ** 0.5, L=lib)
        return run, nl, None

    return rig.columns(make, lambda s, n: {"us_per_layer": round(s / n * 1e6, 2), "GBps": round(b * n / s / 1e9, 2),
                                           "working_set_MB": round(nl * per / 1e6, 1)})


def mla(torch, K, ctx, stream, dev, gen, args, rig=None):
    """Absorbed latent attention (model/deepseek.rs:553-591) at DeepSeek-V2-Lite
    geometry: 16 heads, latent 512, rope 64, over nl layers of distinct caches
    ~ N(0, 1); bytes = every cached row (576 floats) read once, plus the
    queries and the output; flops 4 * 16 * (576 + 512) / 2 * L per layer."""
    H = 16
    res = {}
    for L in (1024, 8192, 32768):
        nl = max(8, min(32, -(-600 * 2**20 // (4 * L * 576))))  # past 2x the 256 MB cache from L = 8192
        c = torch.randn(nl, L, 512, device=dev, generator=gen)
        pe = torch.randn(nl, L, 64, device=dev, generator=gen)
        ql = torch.randn(H * 512, device=dev, generator=gen)
        qp = torch.randn(H * 64, device=dev, generator=gen)
        o = torch.empty(H * 512, device=dev)

        def run():
            for l in range(nl):
                K.mla_attend_dev(ctx, H, ql.data_ptr(), qp.data_ptr(), c[l].data_ptr(), pe[l].data_ptr(), L,
                                 1.0 / 192 ** 0.5, o.data_ptr())

        g = Graph(torch, ctx, stream, run)
        s = g.time(max(5, args.steps // 5), 2) / nl
        b = 4 * L * 576 + 4 * H * (512 + 64 + 512)
        res[str(L)] = {"us_per_layer": round(s * 1e6, 2), "GBps": round(b / s / 1e9, 1),
                       "TFLOPS": round(2 * H * (576 + 512) * L / s / 1e12, 2), "layers": nl,
                       "memory": "HBM" if nl * 4 * L * 576 > 2 * 256 * 2**20 else "cache-resident (<= 2x 256 MB)"}
        del g, c, pe
        if rig is not None and L == 32768:
            res[str(L)]["cpu"] = mla_cpu(rig, H, L)
    log(f"mla: {res}")
    return res


def write_q8_cache(path, n_mats, rows, cols, sc, qs):
    """A cache file of n_mats copies of one q8 matrix, written a array at a
    time: the container of crates/llm/src/qcache.rs:932-1040 (magic, 56
    reserved bytes, each array on a 64-byte boundary named by an
    [offset, count] span, the JSON header after the last array, its offset as
    a little-endian u64 at the end), with the CPU engine's q8 entries
    (qcache.rs:986-1005)."""
    import json
    import struct

    tensors = {}
    with open(path, "wb") as f:
        f.write(b"NANOQ\x00\x00\x01" + bytes(56))
        at = 64

        def put(a):
            nonlocal at
            pad = (64 - at % 64) % 64
            f.write(bytes(pad))
            at += pad
            span = [at, int(a.size)]
            f.write(a.tobytes())
            at += a.nbytes
            return span

        for i in range(n_mats):
            tensors[f"m{i}"] = {"kind": "q8", "shape": [rows, cols], "scales": put(sc), "qs": put(qs)}
        header = {"version": 2, "precision": "q8", "repo": "bench/synthetic", "tensors": tensors}
        f.write(json.dumps(header).encode() + struct.pack("<Q", at))


def qcache_upload(K, ctx, n_mats=16, rows=14336, cols=4096):
    """The load path of crates/llm/src/qcache.rs onto the device: a cache file
    of n_mats q8 matrices (Llama-3-8B gate shape, 0.99 GB) written once, then
    every matrix uploaded from the mapped file (page cache, as on any load
    after the first) through pinned staging; beside it the same arrays
    uploaded from ordinary host memory by kh_weight_q8."""
    import tempfile

    rng = np.random.default_rng(0)
    qs = rng.integers(-127, 128, rows * cols, dtype=np.int8)
    sc = rng.random(rows * cols // 32, dtype=np.float32) * 1e-3
    nbytes = n_mats * (qs.nbytes + sc.nbytes)
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "bench.nanoq"
        write_q8_cache(path, n_mats, rows, cols, sc, qs)
        qc = K.QCache(path)
        for i in range(2):  # warm: page cache and allocator
            qc.weight(ctx, f"m{i}")
        t = time.perf_counter()
        ws = [qc.weight(ctx, f"m{i}") for i in range(n_mats)]
        t_qc = time.perf_counter() - t
        del ws
        t = time.perf_counter()
        ws = [K.Weight.from_q8(ctx, rows, cols, sc, qs) for _ in range(n_mats)]
        t_host = time.perf_counter() - t
        del ws
        qc.close()
    res = {"bytes": nbytes, "qcache_GBps": round(nbytes / t_qc / 1e9, 2),
           "pageable_host_GBps": round(nbytes / t_host / 1e9, 2), "matrices": n_mats,
           "shape": f"{rows}x{cols} q8"}
    log(f"qcache upload: {res}")
    return res


def q8_ffn_cpu(rig, qlayers, fb):
    """Weight::matvec_bt's q8 path (QActivation, qrow per row, quant.rs:410-512)
    on the host over the same 72 FFN matrices (copied back from the device,
    354.7 MB), one call each, as the device figure beside it."""
    O = rig.O
    mats = []
    for L in qlayers:
        for name, (rows, cols) in (("gate", (4864, 896)), ("up", (4864, 896)), ("down", (896, 4864))):
            s8, q8 = L[name].parts()
            mats.append((s8, q8, rows, cols, L["m" if name == "down" else "h"].cpu().numpy()))

    def make(lib, nt):
        def run():
            for s8, q8, rows, cols, x in mats:
                O.matvec_q8(s8, q8, rows, cols, x, L=lib)
        return run, len(mats), None

    return rig.columns(make, lambda s, n: {"us_per_gemv": round(s / n * 1e6, 2), "GBps": round(fb / s / 1e9, 2)})


def q8_qwen(torch, K, ctx, stream, dev, gen, args, rig=None):
    """Q8 GEMV at Qwen2.5-0.5B decode shapes, 24 layers
    of distinct weights plus the 151936x896 lm_head."""
    out = {}
    qwen = {"q": (896, 896), "k": (128, 896), "v": (128, 896), "o": (896, 896),
            "gate": (4864, 896), "up": (4864, 896), "down": (896, 4864)}
    qlayers = []
    with torch.cuda.stream(stream):
        for l in range(24):
            L = {}
            for name, (rows, cols) in qwen.items():
                f = torch.randn(rows, cols, device=dev, generator=gen) * 0.02
                L[name] = K.Weight.quantize_dev(ctx, rows, cols, f.data_ptr(), K.Q8)
                L["y_" + name] = torch.empty(rows, device=dev)
            for name, n in (("x", 896), ("a", 896), ("h", 896), ("m", 4864)):
                L[name] = torch.randn(n, device=dev, generator=gen)
            qlayers.append(L)
        f = torch.randn(151936, 896, device=dev, generator=gen) * 0.02
        head = K.Weight.quantize_dev(ctx, 151936, 896, f.data_ptr(), K.Q8)
        heads = [head]
        for _ in range(3):  # four copies in turn: 615 MB, past twice the 256 MB cache
            f = torch.randn(151936, 896, device=dev, generator=gen) * 0.02
            heads.append(K.Weight.quantize_dev(ctx, 151936, 896, f.data_ptr(), K.Q8))
        del f
        xh = torch.randn(896, device=dev, generator=gen)
        yh = torch.empty(151936, device=dev)
    torch.cuda.synchronize()
    qbytes = 24 * sum(q8_bytes(r, c) for r, c in qwen.values()) + q8_bytes(151936, 896)

    def many(ws, xs, ys):
        n = len(ws)
        arr = lambda vals: (K.C.c_void_p * n)(*vals)
        assert K.lib.kh_matvec_many_dev(ctx.h, n, arr([w.h.value for w in ws]), arr(xs), arr(ys)) == 0

    def step():
        for L in qlayers:
            many([L["q"], L["k"], L["v"]], [L["x"].data_ptr()] * 3,
                 [L["y_q"].data_ptr(), L["y_k"].data_ptr(), L["y_v"].data_ptr()])
            L["o"].matvec_bt_dev(L["a"].data_ptr(), L["y_o"].data_ptr())
            many([L["gate"], L["up"]], [L["h"].data_ptr()] * 2, [L["y_gate"].data_ptr(), L["y_up"].data_ptr()])
            L["down"].matvec_bt_dev(L["m"].data_ptr(), L["y_down"].data_ptr())
        head.matvec_bt_dev(xh.data_ptr(), yh.data_ptr())

    g = Graph(torch, ctx, stream, step)
    s = g.time(args.steps, args.warmup)
    out["q8_qwen05b_decode_gemvs"] = {"GBps": round(qbytes / s / 1e9, 1), "us_per_token": round(s * 1e6, 2),
                                      "bytes_per_token": qbytes, "launches": 24 * 4 + 1}
    del g

    def head_only():
        for i in range(8):
            heads[i & 3].matvec_bt_dev(xh.data_ptr(), yh.data_ptr())

    g = Graph(torch, ctx, stream, head_only)
    s = g.time(args.steps, args.warmup) / 8
    out["q8_lm_head_151936x896"] = {"GBps": round(q8_bytes(151936, 896) / s / 1e9, 1), "us": round(s * 1e6, 2),
                                    "rotation": f"4 copies, {4 * q8_bytes(151936, 896) / 1e6:.1f} MB"}
    del g, heads

    def ffn_shapes():
        for L in qlayers:
            for name in ("gate", "up", "down"):
                L[name].matvec_bt_dev(L["m" if name == "down" else "h"].data_ptr(), L["y_" + name].data_ptr())

    g = Graph(torch, ctx, stream, ffn_shapes)
    s = g.time(args.steps, args.warmup)
    fb = 24 * (2 * q8_bytes(4864, 896) + q8_bytes(896, 4864))
    out["q8_qwen05b_ffn_single_launches"] = {"GBps": round(fb / s / 1e9, 1), "us_per_gemv": round(s / 72 * 1e6, 2),
                                             "rotation": f"72 matrices, {fb / 1e6:.1f} MB"}
    del g
    if rig is not None:
        out["q8_qwen05b_ffn_single_launches"]["cpu"] = q8_ffn_cpu(rig, qlayers, fb)

    # the dequantising kernel (Weight::matvec_bt_dequant, quant.rs:522-589)
    # beside the integer path on the same 72 matrices, one launch each
    def ffn_dequant():
        for L in qlayers:
            for name in ("gate", "up", "down"):
                L[name].matvec_bt_dequant_dev(L["m" if name == "down" else "h"].data_ptr(), L["y_" + name].data_ptr())

    g = Graph(torch, ctx, stream, ffn_dequant)
    s = g.time(args.steps, args.warmup)
    out["q8_qwen05b_ffn_dequant_single_launches"] = {"GBps": round(fb / s / 1e9, 1),
                                                     "us_per_gemv": round(s / 72 * 1e6, 2)}
    log(f"q8 qwen: {out}")
    del g
    return out


def attend_cpu(rig, nh, nkv, hd, L):
    """model::attend (mod.rs:769-819, parallel over query heads) on the host:
    per call every layer of `nl` distinct caches (twice the host LLC)."""
    O = rig.O
    kvd = nkv * hd
    per = 2 * 4 * L * kvd
    nl = rig.layers_past_llc(per)
    rng = np.random.default_rng(L + nh)
    ks = rng.standard_normal((nl, L, kvd), dtype=np.float32)
    vs = rng.standard_normal((nl, L, kvd), dtype=np.float32)
    q = rng.standard_normal(nh * hd, dtype=np.float32)
    b = per + 8 * nh * hd

    def make(lib, nt):
        def run():
            for l in range(nl):
                O.attend(nh, nkv, hd, q, ks[l], vs[l], L, L=lib)
        return run, nl, None

    return rig.columns(make, lambda s, n: {"us_per_layer": round(s / n * 1e6, 2), "GBps": round(b * n / s / 1e9, 2),
                                           "working_set_MB": round(nl * per / 1e6, 1)})


def attend(torch, K, ctx, stream, dev, gen, args, rig=None):
    """GQA decode attention at Qwen2.5-0.5B geometry
    (14 query heads, 2 KV heads, head_dim 64) over 24 layers of distinct f32
    caches ~ N(0, 1); bytes = each K and V row read once, plus q and out."""
    att = {}
    # (heads, kv heads, head dim, layers of distinct caches per length): at
    # least 24 layers, and past 2x the 256 MB cache where a layer allows it
    # (64 at Qwen L = 8192); smaller caches are cache-resident and labelled so
    for geom, lengths in (((14, 2, 64), (1024, 8192, 32768)), ((32, 8, 128), (128, 512, 2048, 8192))):
        nh, nkv, hd = geom
        spec = K.Spec(nh, nkv, hd)
        kvd = nkv * hd
        res = {}
        for L in lengths:
            per = 2 * 4 * L * kvd
            nl = max(24 if nh == 14 else 32, min(72, -(-600 * 2**20 // per)))
            kv = torch.randn(nl, 2, L, kvd, device=dev, generator=gen)
            q = torch.randn(nh * hd, device=dev, generator=gen)
            o = torch.empty(nh * hd, device=dev)

            def run():
                for l in range(nl):
                    K.attend_dev(ctx, spec, q.data_ptr(), kv[l, 0].data_ptr(), kv[l, 1].data_ptr(), L, o.data_ptr())

            g = Graph(torch, ctx, stream, run)
            s = g.time(max(5, args.steps // 5), 2) / nl
            b = per + 8 * nh * hd
            res[str(L)] = {"us_per_layer": round(s * 1e6, 2), "GBps": round(b / s / 1e9, 1), "layers": nl,
                           "cache_MB": round(nl * per / 1e6, 1),
                           "memory": "HBM" if nl * per > 2 * 256 * 2**20 else "cache-resident (<= 2x 256 MB)"}
            del g, kv
            if rig is not None and L >= (8192 if nh == 14 else 2048):  # the lengths the HBM figures are quoted at
                res[str(L)]["cpu"] = attend_cpu(rig, nh, nkv, hd, L)
        att["qwen05b_14_2_64" if nh == 14 else "llama8b_32_8_128"] = res
    log(f"attend: {att}")
    return att


def prefill_cpu(rig, m, k, n, prec):
    """Weight::matmul_bt on the host (the oracle's x86 path: QActBatch, then
    row_dot per row and token, quant.rs:751-907; f32: tensor::gemm_bt's 4 x 4
    register tile, tensor.rs:102-193), with the activation quantisation inside
    the call as the reference has it.  The large shape runs a sample of its
    output rows (and, on one thread, of its tokens): the same loop, fewer rows;
    the (512, 896, 4864) shape runs whole on all threads and at 64 tokens
    (the reference's own m-sweep size) on one."""
    O = rig.O
    rng = np.random.default_rng(m + n)
    big = m * n * k > 4e9
    n_all, n_one = (512, 256) if big else (n, n)
    m_all, m_one = (m, 128) if big else (m, 64)
    w = (rng.standard_normal((n_all, k), dtype=np.float32) * 0.02).ravel()
    xs = rng.standard_normal((m_all, k), dtype=np.float32).ravel()
    wq = O.quantize_q8(w, n_all, k) if prec == "q8" else None

    def make(lib, nt):
        mm, nn = (m_all, n_all) if nt > 1 else (m_one, n_one)
        x = xs[:mm * k]
        if prec == "q8":
            s8, q8 = wq
            s8, q8 = s8[:nn * k // 32], q8[:nn * k]
            run = lambda: O.matmul_q8(s8, q8, nn, k, x, mm, L=lib)
        else:
            wf = w[:nn * k]
            run = lambda: O.matmul_f32(wf, nn, k, x, mm, L=lib)
        note = None if (mm, nn) == (m, n) else f"{mm} tokens x {nn} of {n} output rows"
        return run, 2 * mm * nn * k, note

    return rig.columns(make, lambda s, ops: {"GOPS": round(ops / s / 1e9, 2), "ms_per_call": round(s * 1e3, 3)})


def prefill(torch, K, ctx, stream, dev, gen, args, rig=None):
    """batched-prefill GEMM, q8 (int8 MFMA) and f32
    (f32 MFMA), at (M, K, N) = (512, 896, 4864) and (2048, 4096, 14336).
    Each call is Weight::matmul_bt on device pointers: the activation
    quantiser plus the GEMM, y[M, N] f32."""
    res = {}
    for (m, k, n) in ((512, 896, 4864), (2048, 4096, 14336)):
        f = torch.randn(n, k, device=dev, generator=gen) * 0.02
        xs = torch.randn(m, k, device=dev, generator=gen)
        y = torch.empty(m, n, device=dev)
        ops = 2 * m * n * k
        for prec, code in (("q8", K.Q8), ("f32", K.F32)):
            with torch.cuda.stream(stream):
                w = K.Weight.quantize_dev(ctx, n, k, f.data_ptr(), code)
            torch.cuda.synchronize()

            def run():
                for _ in range(4):
                    w.matmul_bt_dev(xs.data_ptr(), m, y.data_ptr())

            g = Graph(torch, ctx, stream, run)
            s = g.time(max(5, args.steps // 5), 2, settle=1.0) / 4
            peak = 5000.0 if prec == "q8" else 157.3
            tops = ops / s / 1e12
            res[f"{prec}_{m}x{k}x{n}"] = {"us": round(s * 1e6, 2), "TOPS": round(tops, 2),
                                          "frac_of_mfma_peak": round(tops / peak, 4),
                                          "peak": f"{peak} T{'OP' if prec == 'q8' else 'FLOP'}/s"}
            del g, w
            if rig is not None:
                res[f"{prec}_{m}x{k}x{n}"]["cpu"] = prefill_cpu(rig, m, k, n, prec)
        del f, xs, y
    # the reference's sweep over the batch (docs/engine.md:663-669): mlp.down
    # [896 x 4864], q8, m = 2..128; up to 8 rows take the multi-token GEMV
    n, k = 896, 4864
    f = torch.randn(n, k, device=dev, generator=gen) * 0.02
    with torch.cuda.stream(stream):
        w = K.Weight.quantize_dev(ctx, n, k, f.data_ptr(), K.Q8)
    torch.cuda.synchronize()
    sweep = {}
    for m in (2, 8, 32, 64, 128):
        xs = torch.randn(m, k, device=dev, generator=gen)
        y = torch.empty(m, n, device=dev)

        def run():
            for _ in range(8):
                w.matmul_bt_dev(xs.data_ptr(), m, y.data_ptr())

        g = Graph(torch, ctx, stream, run)
        s = g.time(max(5, args.steps // 5), 2, settle=0.3) / 8
        sweep[str(m)] = {"us": round(s * 1e6, 2), "GMACps": round(m * n * k / s / 1e9, 1),
                         "TOPS": round(2 * m * n * k / s / 1e12, 2),
                         "path": "multi-token GEMV" if m <= 8 else "int8 MFMA GEMM",
                         "vs_reference_smmla_q8_GMACps": {2: 77.9, 8: 153.6, 32: 285.4, 64: 306.3, 128: 319.7}[m]}
        del g, xs, y
    res["q8_m_sweep_mlp_down_896x4864"] = sweep
    del f, w
    log(f"prefill gemm: {res}")
    return res


def moe(torch, K, ctx, stream, dev, gen, args, n_layers=8, rig=None):
    """a DeepSeek-V2-Lite MoE layer at q8 (hidden 2048,
    64 experts of width 1408 + a fused shared expert of width 2816, top-6
    softmax routing).  Decode: one token through n_layers distinct layers
    (weights ~ N(0, 0.02), router ~ N(0, 0.5), x ~ N(0, 1) per layer), HIP
    graph; bytes = the router, the shared expert and the six chosen experts'
    weights read once.  Prefill: 512 tokens through one layer, 2*M*N*K ops."""
    hidden, inter, n_exp, k, sh = 2048, 1408, 64, 6, 2816
    res = {}

    def q8(rows, cols, sd=0.02):
        f = torch.randn(rows, cols, device=dev, generator=gen) * sd
        return K.Weight.quantize_dev(ctx, rows, cols, f.data_ptr(), K.Q8)

    layers = []
    first = None  # layer 0's weights, for the host's copy
    with torch.cuda.stream(stream):
        for _ in range(n_layers):
            m = K.Moe(ctx, n_exp, k, hidden, inter)
            ws = {"router": q8(n_exp, hidden, 0.5), "experts": [], "shared": None}
            m.set_router(ws["router"])
            for x in range(n_exp):
                e3 = (q8(inter, hidden), q8(inter, hidden), q8(hidden, inter))
                m.set_expert(x, *e3)
                ws["experts"].append(e3)
            ws["shared"] = (q8(sh, hidden), q8(sh, hidden), q8(hidden, sh))
            m.set_shared(*ws["shared"])
            first = first or ws
            layers.append((m, torch.randn(hidden, device=dev, generator=gen), torch.empty(hidden, device=dev)))
    torch.cuda.synchronize()

    def q8b(r, c):
        return r * c + 4 * r * c // 32

    tok_bytes = q8b(n_exp, hidden) + 3 * q8b(sh, hidden) + k * 3 * q8b(inter, hidden) + 8 * hidden

    def decode():
        for m, x, y in layers:
            m.run_dev(x.data_ptr(), 1, y.data_ptr())

    g = Graph(torch, ctx, stream, decode)
    s = g.time(max(5, args.steps // 5), 2) / n_layers
    res["decode_1tok"] = {"us_per_layer": round(s * 1e6, 2), "GBps": round(tok_bytes / s / 1e9, 1),
                          "bytes_per_layer": tok_bytes, "launches_per_layer": 5}
    del g
    m0 = layers[0][0]
    M = 512
    hs = torch.randn(M, hidden, device=dev, generator=gen)
    ys = torch.empty(M, hidden, device=dev)

    def pre():
        m0.run_dev(hs.data_ptr(), M, ys.data_ptr())

    g = Graph(torch, ctx, stream, pre)
    s = g.time(max(5, args.steps // 5), 2, settle=1.0)
    ops = 2 * M * k * 3 * inter * hidden + 2 * M * 3 * sh * hidden
    # 512 tokens x k picks over n_exp experts pick every expert (about 48
    # rows each), so the layer reads every expert's weights once: HBM-bound
    # (651 MB at 8 TB/s = 81 us against 71 G int8 ops at 5 POP/s = 14 us)
    pre_bytes = q8b(n_exp, hidden) + 3 * q8b(sh, hidden) + n_exp * 3 * q8b(inter, hidden) + 8 * M * hidden
    res["prefill_512tok"] = {"us": round(s * 1e6, 1), "TOPS": round(ops / s / 1e12, 2), "ops": ops,
                             "GBps": round(pre_bytes / s / 1e9, 1), "bytes": pre_bytes, "bound": "hbm"}
    del g
    if rig is not None:
        moe_cpu(rig, res, first, m0, hidden, inter, n_exp, k, sh, tok_bytes, ops)
    log(f"moe: {res}")
    return res


def moe_cpu(rig, res, ws, dev_layer, hidden, inter, n_exp, top_k, sh, tok_bytes, ops512):
    """Moe::run (ffn.rs:615-708, the oracle's restatement) on the host with
    layer 0's weights copied back from the device (0.64 GB): decode over 16
    tokens in turn (each routes to its own six experts, so the calls stream
    most of the layer), and the 512-token prefill (64 tokens on one thread).
    A parity spot check of the device layer against it rides along."""
    O = rig.O
    cat = lambda i: tuple(np.concatenate(a) for a in zip(*[e[i].parts() for e in ws["experts"]]))
    router, gate, up, down = ws["router"].parts(), cat(0), cat(1), cat(2)
    shared = tuple(w.parts() for w in ws["shared"]) + (sh,)
    rng = np.random.default_rng(64)
    toks = rng.standard_normal((512, hidden), dtype=np.float32)

    def layer(x, m, lib):
        return O.moe_run_q8(x, m, hidden, inter, n_exp, top_k, router, gate, up, down, shared=shared, L=lib)

    want = layer(toks[0], 1, rig.native)
    got = dev_layer.run(toks[0], 1)
    res["decode_1tok"]["rel_err_vs_oracle"] = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))

    def make_dec(lib, nt):
        def run():
            for i in range(16):
                layer(toks[i], 1, lib)
        return run, 16, None

    res["decode_1tok"]["cpu"] = rig.columns(make_dec, lambda s, n: {"us_per_layer": round(s / n * 1e6, 1),
                                                                     "GBps": round(tok_bytes * n / s / 1e9, 2)})

    def make_pre(lib, nt):
        mm = 512 if nt > 1 else 64
        run = lambda: layer(toks[:mm], mm, lib)
        return run, ops512 * mm // 512, None if mm == 512 else f"{mm} of the 512 tokens"

    res["prefill_512tok"]["cpu"] = rig.columns(make_pre, lambda s, o: {"GOPS": round(o / s / 1e9, 2),
                                                                        "ms_per_call": round(s * 1e3, 2)})


def qwen05b_session(torch, K, ctx, stream, dev, gen, n_ctx=2048):
    """A device session of Qwen2.5-0.5B's shape, q8 (24 layers, n_embd 896,
    14/2 heads of 64, ffn 4864, vocab 151936, tied embedding, q/k/v biases;
    weights ~ N(0, 0.02), norms 1, RoPE theta 1e6)."""
    spec = dict(n_layer=24, n_embd=896, n_head=14, n_kv_head=2, head_dim=64, n_ff=4864, vocab=151936,
                n_ctx=n_ctx, eps=1e-6, rope_interleaved=0)
    e, qd, kvd, ff = 896, 896, 128, 4864

    def q8(rows, cols):
        f = torch.randn(rows, cols, device=dev, generator=gen) * 0.02
        return K.Weight.quantize_dev(ctx, rows, cols, f.data_ptr(), K.Q8)

    ones = np.ones(e, np.float32)
    layers = []
    with torch.cuda.stream(stream):
        m = K.Llm(ctx, **spec)
        rng = np.random.default_rng(0)
        for l in range(24):
            L = {n: q8(r, c) for n, (r, c) in dict(q=(qd, e), k=(kvd, e), v=(kvd, e), o=(e, qd), gate=(ff, e),
                                                    up=(ff, e), down=(e, ff)).items()}
            L.update(attn_norm=ones, mlp_norm=ones, q_b=(rng.standard_normal(qd) * 0.02).astype(np.float32),
                     k_b=(rng.standard_normal(kvd) * 0.02).astype(np.float32),
                     v_b=(rng.standard_normal(kvd) * 0.02).astype(np.float32))
            m.set_layer(l, *[L[n] for n in ("q", "k", "v", "o", "gate", "up", "down")], ones, ones, L["q_b"],
                        L["k_b"], L["v_b"])
            layers.append(L)
        embed = q8(151936, e)
        m.set_ends(embed, ones)
        half = 32
        inv = 1.0 / (1e6 ** (np.arange(half, dtype=np.float32) * 2.0 / 64))  # Rope::new, tensor.rs:390-407
        ang = np.arange(n_ctx, dtype=np.float32)[:, None] * inv[None, :].astype(np.float32)
        cos_t, sin_t = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
        m.set_rope(cos_t, sin_t, n_ctx)
    torch.cuda.synchronize()

    def host(lib=None):
        """The same model for the oracle (O.Llm), its weights copied back from
        the device (0.51 GB), running its matmuls and attention on `lib`."""
        import oracle as O

        hl = []
        for L in layers:
            d = {n: (L[n].parts() if isinstance(L[n], K.Weight) else L[n]) for n in L}
            hl.append(d)
        return O.Llm(spec, hl, embed.parts(), ones, None, cos_t.ravel(), sin_t.ravel(), L=lib)

    return m, host


def decode(torch, K, ctx, stream, dev, gen, args, n_ctx=2048, warm=32, timed=256, rig=None):
    """The second half of BASELINE.json's metric: Qwen2.5-0.5B-shaped q8
    decode, tokens per second, on the device-resident session
    (qwen05b_session).  Greedy tokens, one HIP graph replay per token; `warm`
    tokens first, then `timed` tokens timed with HIP events on the session's
    stream (context warm..warm+timed)."""
    m, host = qwen05b_session(torch, K, ctx, stream, dev, gen, n_ctx)
    torch.cuda.synchronize()
    first = m.generate(1, warm)  # captures the step's graph
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        m.generate_launch(timed)
        e1.record(stream)
        e1.synchronize()
    s = e0.elapsed_time(e1) / 1e3
    tps = timed / s
    res = {"tok_per_s": round(tps, 1), "ms_per_token": round(s / timed * 1e3, 4), "context": [warm, warm + timed],
           # per layer q/k/v, attention, o, gate+up, down; past 256 positions
           # the attention is split and merged (one launch more per layer);
           # plus the head, whose workgroups keep their greedy choices and
           # whose last to finish takes the best, advances the step and writes
           # the next token's embedding row
           "launches_per_token": {"positions <= 256": 24 * 5 + 1, "positions > 256": 24 * 6 + 1},
           "vs_reference_cpu_q8_112tps": round(tps / 112.0, 2),
           "vs_reference_metal_q8_191tps": round(tps / 191.0, 2), "first_tokens": [int(t) for t in first[:4]]}
    log(f"qwen0.5b q8 decode: {res}")
    ref = None
    if rig is not None:
        ref = host(rig.native)
        m.truncate(0)
        got, _ = m.forward(1)
        want = ref.forward(1)
        res["rel_err_vs_oracle_first_token"] = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
        res["cpu"] = session_cpu(rig, host, ref)
    res["prefill"] = prefill_session(m, rig=rig, host=host, ref=ref)
    res["batched"] = decode_batched(torch, m, warm)
    m.free()
    return res


def session_cpu(rig, host, ref):
    """The oracle's decoder (O.Llm: the forward of llama.rs:224-289 and the
    head, sequenced in Python over the oracle's C kernels) on the host, one
    token a call, over the same weights as the device session; the native
    build's model is `ref`, the portable one is built here."""
    models = {"native": ref}
    if len(rig.builds) > 1:
        models["portable"] = host(rig.builds[0][1])
    else:
        models = {"portable": ref}

    def make(lib, nt):
        mdl = models["native" if lib is rig.native and "native" in models else "portable"]

        def run():
            if mdl.len >= 1500:
                mdl.len = 0
            mdl.forward(7)
        return run, 1, None

    return rig.columns(make, lambda s, n: {"tok_per_s": round(n / s, 2), "ms_per_token": round(s / n * 1e3, 2)})


def prefill_session(m, n=640, reps=5, rig=None, host=None, ref=None):
    """A prompt read on the device (Session::forward(&[u32]), mod.rs:842): n
    tokens from an empty cache, in passes of prefill_pass tokens (Rows::Following,
    llama.rs:224-289: the projections on the int8 GEMM, every row's attention
    causal over the held cache; the default pass, 512, cuts 640 into 512 + 128),
    host to host: tokens up, last logits and the
    next token back.  Each pass size is timed as the best of `reps` calls after
    one untimed call that captures its passes; beside it the same prompt fed
    one token at a time (kh_llm_forward per token, as the device read prompts
    before), and the reference's published 640-token prefill at
    Qwen2.5-0.5B q8 on the M5 Pro CPU: 1.20 s with SMMLA, 6.20 s token at a
    time (docs/engine.md:587-596)."""
    prompt = (np.arange(n, dtype=np.int64) * 7919 + 11) % 151936
    out = {"tokens": n, "reference_m5pro_cpu_s": {"smmla_passes": 1.20, "token_at_a_time": 6.20}}
    for chunk in (64, 128, 256, 512, 640):  # 512: the default (the reference GPU backend's pass)
        m.reading(chunk)
        m.truncate(0)
        m.forward_tokens(prompt, want_logits=False)
        best = float("inf")
        for _ in range(reps):
            m.truncate(0)
            t0 = time.perf_counter()
            m.forward_tokens(prompt, want_logits=True)
            best = min(best, time.perf_counter() - t0)
        out[f"chunk_{chunk}"] = {"ms": round(best * 1e3, 3), "tok_per_s": round(n / best, 1),
                                 "passes": -(-n // chunk)}
    m.reading(0)
    m.truncate(0)
    m.forward(int(prompt[0]), want_logits=False)
    m.truncate(0)
    t0 = time.perf_counter()
    for t in prompt:
        m.forward(int(t), want_logits=False)
    s = time.perf_counter() - t0
    out["token_at_a_time"] = {"ms": round(s * 1e3, 3), "tok_per_s": round(n / s, 1)}
    out["default_chunk"] = m.prefill_pass(1 << 20)
    d = out[f"chunk_{out['default_chunk']}"]["ms"] / 1e3
    out["vs_reference_smmla"] = round(1.20 / d, 1)
    m.truncate(0)
    if rig is not None and host is not None:
        # the oracle's forward_tokens (Rows::Following over the oracle's
        # matmuls, passes of 64 as the CPU session reads, mod.rs:1004-1006);
        # all threads: 128 of the 640 tokens, one thread: 64
        ref = ref if ref is not None else host(rig.native)
        native_only = [b for b in rig.builds if b[1] is rig.native]

        def make(lib, nt):
            k = 128 if nt > 1 else 64

            def run():
                ref.len = 0
                ref.forward_tokens(prompt[:k], chunk=64)
            return run, k, f"{k} of the {n} tokens"

        out["cpu"] = rig.columns(make, lambda s, k: {"tok_per_s": round(k / s, 1),
                                                     "s_for_640_at_this_rate": round(n * s / k, 2)},
                                 builds=native_only)
        ref.len = 0
    log(f"qwen0.5b q8 prefill: {out}")
    return out


def decode_batched(torch, m, warm, steps=20):
    """Batched decode (Session::forward_each, mod.rs:1190-1202; llama.rs:418-434)
    on the same session: B conversations of `warm` + b tokens each, parked,
    then advanced together one token per call, greedy (each row's next token
    fed back).  Each call is host to host: the tables up, one captured pass
    for B rows, the next tokens back.  Timed over `steps` calls after two
    untimed calls (the capture, then a first replay, which can pay one-off
    costs) with the host clock."""
    out = {}
    m.truncate(0)  # the timed single-token run left its conversation in the session
    for B in (2, 4, 8, 16, 32):
        parked = []
        for b in range(B):
            m.generate(1 + b, warm + b)  # row b: warm + b positions
            parked.append(m.park())
        _, toks = m.forward_each(np.arange(B, dtype=np.int32), parked, want_logits=False)
        _, toks = m.forward_each(toks, parked, want_logits=False)
        t0 = time.perf_counter()
        for _ in range(steps):
            _, toks = m.forward_each(toks, parked, want_logits=False)
        s = (time.perf_counter() - t0) / steps
        out[str(B)] = {"ms_per_step": round(s * 1e3, 4), "tok_per_s": round(B / s, 1),
                       "row_context": [warm + 2, warm + B + 1 + steps]}
        for p in parked:
            p.free()
    log(f"qwen0.5b q8 batched decode: {out}")
    return out


def _host_llc_bytes() -> int:
    """The host's last-level cache in bytes, all instances (lscpu), or 0."""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        for line in out.splitlines():
            if line.startswith("L3 cache"):
                v = line.split(":", 1)[1].strip()      # e.g. "105 MiB (1 instance)"
                num, unit = v.split()[0], v.split()[1]
                scale = {"KiB": 1 << 10, "MiB": 1 << 20, "GiB": 1 << 30}.get(unit, 1 << 20)
                return int(float(num) * scale)
    except Exception:
        pass
    return 0


def _native_oracle(tmpdir: str):
    """The oracle compiled on this host with -march=native (the box's own CPU,
    which the development container's build cannot target)."""
    import ctypes

    import oracle as O

    out = Path(tmpdir) / "libkvad_oracle_native.so"
    cmd = ["gcc", "-O3", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-fPIC", "-march=native",
           "-shared", "-o", str(out), str(ROOT / "oracle" / "kvad_oracle.c"), "-lm"]
    subprocess.run(cmd, check=True, capture_output=True)
    return O._declare(ctypes.CDLL(str(out)))


def _calibrated(fn, budget_s: float):
    """bench_matvec.rs:24-50's protocol: three warm-ups (one when a call takes
    more than 50 ms), an iteration count calibrated to about 0.1 s a round
    (at least one call: a call over these working sets can take longer), best
    of five rounds; stops early when the column's time budget is spent.
    Seconds per call, rounds run."""
    t_end = time.perf_counter() + budget_s
    t = time.perf_counter()
    fn()
    if time.perf_counter() - t < 0.05:
        fn()
        fn()
    t = time.perf_counter()
    fn()
    one = max(time.perf_counter() - t, 1e-9)
    iters = max(1, min(20000, int(0.1 / one)))
    best, rounds = one, 0
    while rounds < 5 and (rounds == 0 or time.perf_counter() < t_end):
        t = time.perf_counter()
        for _ in range(iters):
            fn()
        best = min(best, (time.perf_counter() - t) / iters)
        rounds += 1
    return best, rounds


class CpuRig:
    """The reference's CPU path restated (the oracle's C), timed on this
    host's cores beside each device figure, in the same run: the portable
    build (-O3, baseline x86-64, the reference's default target) and
    -march=native, each on one thread and on all of the process's threads,
    with bench_matvec.rs:24-50's protocol (_calibrated) under a per-column
    time budget.  Working sets exceed the host's last-level cache where the
    shape allows; a workload too long for the budget at one thread runs a
    stated sample of itself (ops per second are what the columns compare)."""

    def __init__(self, budget_s: float):
        import tempfile

        import oracle as O

        self.O = O
        self.tmp = tempfile.TemporaryDirectory()
        try:
            native = _native_oracle(self.tmp.name)
        except Exception as e:  # no compiler on this host: the portable columns only
            log(f"cpu oracle: no -march=native build ({e})")
            native = None
        self.builds = [("portable", O.lib)] + ([("native", native)] if native is not None else [])
        self.native = native if native is not None else O.lib
        self.threads = O.threads()
        self.budget = budget_s
        self.llc = _host_llc_bytes()

    def columns(self, make, fmt, builds=None):
        """make(lib, threads) -> (call, units per call, sample note or None);
        fmt(seconds per call, units) -> the column's figures."""
        cols = {}
        for bname, lib in self.builds if builds is None else builds:
            for nt in (1, self.threads):
                lib.kvo_set_threads(nt)
                fn, units, note = make(lib, nt)
                sec, rounds = _calibrated(fn, self.budget)
                col = fmt(sec, units)
                col.update(threads=nt, rounds=rounds)
                if note:
                    col["sample"] = note
                cols[f"{bname}_{nt}t"] = col
            lib.kvo_set_threads(self.threads)
        cols["host"] = {"cpu": cpu_model(), "threads": self.threads, "llc_MiB": round(self.llc / 2**20, 1)}
        return cols

    def layers_past_llc(self, per_layer: int, lo: int = 1, hi: int = 64) -> int:
        """Distinct copies that make a working set of twice the host LLC."""
        need = 2 * max(self.llc, 32 << 20)
        return max(lo, min(hi, -(-need // max(per_layer, 1))))


def cpu_baseline(layers, budget_s: float, rig: "CpuRig"):
    """The reference's CPU path restated (the oracle), timed on this host's
    cores: the Q4_K GEMV over the bench's own Llama-3-8B layers (the loop that
    decodes scales once per sub-block, equal to the oracle to the bit), and
    the q8 GEMV (Weight::matvec_bt's integer path) on Qwen2.5-0.5B's lm_head
    shape, the reference's published CPU figure.  Columns: portable build
    (-O3, baseline x86-64) and -march=native, each on one thread and on all
    of the process's threads.  Working sets: one layer (123 MB) on one thread
    and eight layers (985 MB) on all threads, so every thread group's share
    exceeds its last-level cache; q8 likewise over 1 and 7 copies of the
    153 MB head."""
    import numpy as np

    import oracle as O

    names = ["q", "k", "v", "o", "gate", "up", "down"]
    inputs = {"q": "x", "k": "x", "v": "x", "o": "a", "gate": "h", "up": "h", "down": "m"}
    nl_all = min(8, len(layers))
    parts = [{n: L[n].parts()[1] for n in names} for L in layers[:nl_all]]
    xs = [{n: L[inputs[n]].cpu().numpy() for n in names} for L in layers[:nl_all]]
    threads = O.threads()
    per_col = max(2.0, budget_s / 6)
    cols = {}
    builds = rig.builds

    def q4k_pass(lib, nl):
        def run():
            for i in range(nl):
                for n in names:
                    rows, cols_ = LLAMA_LAYER[n]
                    O.matvec_q4k_fast(parts[i][n], rows, cols_, xs[i][n], L=lib)
        return run

    layer_bytes = sum(q4k_bytes(*LLAMA_LAYER[n]) for n in names)
    for bname, lib in builds:
        for nt, nl in ((1, 1), (threads, nl_all)):
            lib.kvo_set_threads(nt)
            sec, rounds = _calibrated(q4k_pass(lib, nl), per_col)
            cols[f"q4k_{bname}_{nt}t"] = {"GBps": round(nl * layer_bytes / sec / 1e9, 2), "threads": nt,
                                          "working_set_MB": round(nl * layer_bytes / 1e6, 1), "rounds": rounds}
        lib.kvo_set_threads(threads)

    # q8: the lm_head shape, host-side weights ~ N(0, 0.02)
    hr, hc = 151936, 896
    s8, q8 = O.quantize_q8(O.normal(900, hr * hc, 0.02), hr, hc)
    heads = [(s8, q8)] + [(s8.copy(), q8.copy()) for _ in range(6)]  # distinct memory, same values
    xh = O.normal(950, hc)
    head_bytes = q8_bytes(hr, hc)
    for bname, lib in builds:
        for nt, nh in ((1, 1), (threads, len(heads))):
            lib.kvo_set_threads(nt)

            def run(lib=lib, nh=nh):
                for s8, q8 in heads[:nh]:
                    O.matvec_q8(s8, q8, hr, hc, xh, L=lib)
            sec, rounds = _calibrated(run, per_col / 2)
            cols[f"q8_lm_head_{bname}_{nt}t"] = {"GBps": round(nh * head_bytes / sec / 1e9, 2), "threads": nt,
                                                 "ms_per_call": round(sec / nh * 1e3, 3),
                                                 "working_set_MB": round(nh * head_bytes / 1e6, 1),
                                                 "rounds": rounds}
        lib.kvo_set_threads(threads)
    del heads

    # parity spot check: the oracle and the device on the same weights and input
    y0 = O.matvec_q4k(parts[0]["o"], 4096, 4096, xs[0]["o"])
    yd = layers[0]["o"].matvec_bt(xs[0]["o"])
    agree = float(np.max(np.abs(y0 - yd)) / max(np.max(np.abs(y0)), 1e-30))
    best_key = max((k for k in cols if k.startswith("q4k_") and not k.endswith("_1t")),
                   key=lambda k: cols[k]["GBps"])
    log(f"cpu oracle ({threads} threads): {cols}; device-vs-oracle rel err {agree:.2e}")
    return {"value": cols[best_key]["GBps"], "unit": "GB/s", "cores": cols[best_key]["threads"], "kind": "port",
            "sample": f"oracle Q4_K GEMV (scales decoded once per sub-block) over {nl_all} of the bench's Llama-3-8B "
                      f"layers ({nl_all * layer_bytes / 1e6:.0f} MB, beyond the host's "
                      f"{_host_llc_bytes() / 2**20:.0f} MiB last-level cache), calibrated rounds, best of up to 5; "
                      f"the value is the {best_key} column",
            "cpu": cpu_model(), "columns": cols, "rel_err_vs_device": agree}


if __name__ == "__main__":
    sys.exit(main())

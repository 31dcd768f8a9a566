"""Writes the golden fixtures in this directory from the CPU oracle.

Each fixture holds a case's inputs and the oracle's outputs, so that
tests/test_golden.py catches any change to the oracle's arithmetic and
tests/test_gpu_golden.py checks the device path against the same vectors.
Inputs come from the restated nervus generator (crates/nervus/src/rng.rs),
seeded per tensor; shapes are small so the files stay a few KB.

    python tests/golden/make_golden.py     # rewrites tests/golden/*.npz
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

import oracle as O  # noqa: E402


def quant_cases() -> dict:
    rows, cols = 37, 96
    w = O.normal(1, rows * cols, 0.02)
    w[32:64] = 0.0            # an all-zero block
    w[100] = 3.0              # an outlier
    s8, q8 = O.quantize_q8(w, rows, cols)
    s4, q4 = O.quantize_q4(w, rows, cols)
    rk, ck = 5, 512
    wk = O.normal(2, rk * ck, 0.02)
    wk[:256] *= 10.0          # a super-block at another scale
    bk = O.quantize_q4k(wk, rk, ck)
    x = O.normal(3, cols)
    x[:32] *= 1000.0
    x[64:96] = 0.0
    xq, xs, xsum = O.qact(x)
    xk = O.normal(4, ck)
    xkq, _, _ = O.qact(xk)
    return dict(
        w=w, rows=rows, cols=cols, q8_scales=s8, q8_qs=q8, q4_scales=s4, q4_qs=q4,
        wk=wk, rk=rk, ck=ck, q4k_blocks=bk,
        x=x, x_qs=xq, x_scales=xs, x_sums=xsum, xk=xk,
        dots_q8=O.block_dots_q8(q8, rows, cols, xq),
        dots_q4=O.block_dots_q4(q4, rows, cols, xq, xsum),
        dots_q4k=O.block_dots_q4k(bk, rk, ck, xkq),
        row_q8=np.stack([O.row_q8(s8, q8, cols, r) for r in (0, 1, rows - 1)]),
        row_q4=np.stack([O.row_q4(s4, q4, cols, r) for r in (0, 1, rows - 1)]),
        row_q4k=np.stack([O.row_q4k(bk, ck, r) for r in (0, 2, rk - 1)]),
    )


def gemv_cases() -> dict:
    rows, cols = 37, 96
    w = O.normal(11, rows * cols, 0.02)
    s8, q8 = O.quantize_q8(w, rows, cols)
    s4, q4 = O.quantize_q4(w, rows, cols)
    rk, ck = 9, 512
    wk = O.normal(12, rk * ck, 0.02)
    bk = O.quantize_q4k(wk, rk, ck)
    x = O.normal(13, cols)
    xk = O.normal(14, ck)
    bias = O.normal(15, rows)
    m = 5
    xs = O.normal(16, m * cols)
    xks = O.normal(17, m * ck)
    rf, cf = 7, 13            # f32, a width that is not a multiple of 4
    wf = O.normal(18, rf * cf)
    xf = O.normal(19, cf)
    xfs = O.normal(20, 3 * cf)
    return dict(
        w=w, rows=rows, cols=cols, q8_scales=s8, q8_qs=q8, q4_scales=s4, q4_qs=q4,
        wk=wk, rk=rk, ck=ck, q4k_blocks=bk, x=x, xk=xk, bias=bias, m=m, xs=xs, xks=xks,
        wf=wf, rf=rf, cf=cf, xf=xf, xfs=xfs,
        matvec_q8=O.matvec_q8(s8, q8, rows, cols, x, bias),
        matvec_q4=O.matvec_q4(s4, q4, rows, cols, x, bias),
        matvec_q4k=O.matvec_q4k(bk, rk, ck, xk),
        matvec_f32=O.matvec_f32(w, rows, cols, x, bias),
        matvec_f32_odd=O.matvec_f32(wf, rf, cf, xf),
        matmul_q8=O.matmul_q8(s8, q8, rows, cols, xs, m, bias),
        matmul_q4=O.matmul_q4(s4, q4, rows, cols, xs, m, bias),
        matmul_q4k=O.matmul_q4k(bk, rk, ck, xks, m),
        matmul_f32=O.matmul_f32(w, rows, cols, xs, m, bias),
        matmul_f32_odd=O.matmul_f32(wf, rf, cf, xfs, 3),
        gemm_f32_out_t=O.gemm_f32(xs, m, w, rows, cols),
        matvec_dequant_q8=O.matvec_dequant(1, s8, q8, rows, cols, x),
        matvec_dequant_q4=O.matvec_dequant(2, s4, q4, rows, cols, x),
    )


def attend_cases() -> dict:
    out = {}
    for name, (nh, nkv, hd, L) in {"qwen37": (14, 2, 64, 37), "qwen1": (14, 2, 64, 1),
                                   "llama19": (4, 2, 128, 19), "mha40": (3, 3, 64, 40)}.items():
        q = O.normal(30 + L, nh * hd)
        k = O.normal(31 + L, L * nkv * hd)
        v = O.normal(32 + L, L * nkv * hd)
        out[f"{name}_shape"] = np.array([nh, nkv, hd, L])
        out[f"{name}_q"], out[f"{name}_k"], out[f"{name}_v"] = q, k, v
        out[f"{name}_out"] = O.attend(nh, nkv, hd, q, k, v, L)
    return out


def small_cases() -> dict:
    a, b = O.normal(40, 77), O.normal(41, 77)
    sm = O.normal(42, 50) * 30.0
    x, w = O.normal(43, 96), O.normal(44, 96)
    g, u = O.normal(45, 64), O.normal(46, 64)
    cos_t, sin_t = O.rope_tables(64, 16, 1e6)
    r = O.normal(47, 64)
    return dict(
        a=a, b=b, dot=np.float32(O.dot(a, b)), sm_in=sm, softmax=O.softmax(sm),
        x=x, w=w, rms_norm=O.rms_norm(x, w, 1e-6), gate=g, up=u, swiglu=O.swiglu(g, u),
        rope_cos=cos_t, rope_sin=sin_t, rope_in=r, rope_pos5=O.rope_apply(cos_t, sin_t, 32, r, 5),
        rng_seed42=O.normal(42, 64),
    )


def route_cases() -> dict:
    # ffn.rs:1128-1147 known answer, then V2-Lite-style softmax top-6 of 64,
    # sigmoid + bias + group-limited noaux (V3 style), and group-limited greedy
    kat = np.array([0, 3, 1, -1, 2, 0.5, -2, 4], np.float32)
    lg = O.normal(50, 64)
    bias = O.normal(51, 64, 0.1)
    cases = {
        "kat": (kat, dict(top_k=4, norm_topk=True)),
        "v2lite": (lg, dict(top_k=6)),
        "noaux": (lg, dict(top_k=8, scoring=1, select=2, n_group=8, topk_group=4, norm_topk=True, scale=2.5,
                           bias=bias)),
        "group": (lg, dict(top_k=6, select=1, n_group=8, topk_group=3, norm_topk=False, scale=1.5)),
    }
    out = {"bias": bias}
    for name, (l, kw) in cases.items():
        picks = O.route(l, **kw)
        out[f"{name}_logits"] = l
        out[f"{name}_experts"] = np.array([e for e, _ in picks], np.int32)
        out[f"{name}_weights"] = np.array([w for _, w in picks], np.float32)
    return out


GROUPS = {"quant": quant_cases, "gemv": gemv_cases, "attend": attend_cases, "small": small_cases,
          "route": route_cases}


def main() -> None:
    for name, fn in GROUPS.items():
        data = {k: np.asarray(v) for k, v in fn().items()}
        np.savez_compressed(HERE / f"{name}.npz", **data)
        print(f"wrote {name}.npz ({(HERE / f'{name}.npz').stat().st_size} bytes)")


if __name__ == "__main__":
    main()

"""The device path against the committed golden fixtures (tests/golden/*.npz,
written by the CPU oracle from seeded inputs), through the C ABI.

Bar: quantised codes, scales, block dots and dequantised rows bit-exact;
GEMV/GEMM outputs within 1e-5 x max|ref|; attention within 1e-4 x max|ref|
and exact at one position."""
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

import kvad_amd as K  # noqa: E402

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def close(got, want, rtol):
    scale = max(float(np.max(np.abs(want))), 1e-30)
    err = float(np.max(np.abs(got.astype(np.float64) - want)))
    assert err <= rtol * scale, f"max err {err:.3e} vs scale {scale:.3e}"


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_quantisers_activation_codes_dots_and_rows(ctx):
    g = load("quant")
    rows, cols, rk, ck = int(g["rows"]), int(g["cols"]), int(g["rk"]), int(g["ck"])
    w8 = K.Weight.quantize(ctx, g["w"].reshape(rows, cols), K.Q8)
    s, q = w8.parts()
    np.testing.assert_array_equal(q, g["q8_qs"])
    np.testing.assert_array_equal(bits(s), bits(g["q8_scales"]))
    w4 = K.Weight.quantize(ctx, g["w"].reshape(rows, cols), K.Q4)
    s, q = w4.parts()
    np.testing.assert_array_equal(q, g["q4_qs"])
    np.testing.assert_array_equal(bits(s), bits(g["q4_scales"]))
    wk = K.Weight.quantize(ctx, g["wk"].reshape(rk, ck), K.Q4K)
    np.testing.assert_array_equal(wk.parts()[1], g["q4k_blocks"])
    xq, xs, xsum = K.qact(ctx, g["x"])
    np.testing.assert_array_equal(xq, g["x_qs"])
    np.testing.assert_array_equal(bits(xs), bits(g["x_scales"]))
    np.testing.assert_array_equal(xsum, g["x_sums"])
    np.testing.assert_array_equal(w8.block_dots(g["x"]).ravel(), g["dots_q8"].ravel())
    np.testing.assert_array_equal(w4.block_dots(g["x"]).ravel(), g["dots_q4"].ravel())
    np.testing.assert_array_equal(wk.block_dots(g["xk"]).ravel(), g["dots_q4k"].ravel())
    for i, r in enumerate((0, 1, rows - 1)):
        np.testing.assert_array_equal(bits(w8.row(r)), bits(g["row_q8"][i]))
        np.testing.assert_array_equal(bits(w4.row(r)), bits(g["row_q4"][i]))
    for i, r in enumerate((0, 2, rk - 1)):
        np.testing.assert_array_equal(bits(wk.row(r)), bits(g["row_q4k"][i]))


def test_gemv_and_gemm(ctx):
    g = load("gemv")
    rows, cols, rk, ck, m = (int(g[k]) for k in ("rows", "cols", "rk", "ck", "m"))
    rf, cf = int(g["rf"]), int(g["cf"])
    w8 = K.Weight.from_q8(ctx, rows, cols, g["q8_scales"], g["q8_qs"])
    w4 = K.Weight.from_q4(ctx, rows, cols, g["q4_scales"], g["q4_qs"])
    wk = K.Weight.from_q4k(ctx, rk, ck, g["q4k_blocks"])
    wf = K.Weight.from_f32(ctx, g["w"].reshape(rows, cols))
    wo = K.Weight.from_f32(ctx, g["wf"].reshape(rf, cf))
    close(w8.matvec_bt(g["x"], g["bias"]), g["matvec_q8"], 1e-5)
    close(w4.matvec_bt(g["x"], g["bias"]), g["matvec_q4"], 1e-5)
    close(wk.matvec_bt(g["xk"]), g["matvec_q4k"], 1e-5)
    close(wf.matvec_bt(g["x"], g["bias"]), g["matvec_f32"], 1e-5)
    close(wo.matvec_bt(g["xf"]), g["matvec_f32_odd"], 1e-5)
    close(w8.matmul_bt(g["xs"], m, g["bias"]), g["matmul_q8"], 1e-5)
    close(w4.matmul_bt(g["xs"], m, g["bias"]), g["matmul_q4"], 1e-5)
    close(wk.matmul_bt(g["xks"], m), g["matmul_q4k"], 1e-5)
    close(wf.matmul_bt(g["xs"], m, g["bias"]), g["matmul_f32"], 1e-5)
    close(wo.matmul_bt(g["xfs"], 3), g["matmul_f32_odd"], 1e-5)


@pytest.mark.parametrize("case", ["qwen37", "qwen1", "llama19", "mha40"])
def test_attend(ctx, case):
    g = load("attend")
    nh, nkv, hd, L = (int(v) for v in g[f"{case}_shape"])
    spec = K.Spec(nh, nkv, hd)
    cache = K.KvCache(ctx, 1, nkv * hd, nkv * hd)
    cache.push(0, g[f"{case}_k"], g[f"{case}_v"])
    cache.len = L
    got = K.attend(ctx, spec, g[f"{case}_q"], cache, 0, L)
    if L == 1:
        np.testing.assert_array_equal(got, g[f"{case}_out"])
    else:
        close(got, g[f"{case}_out"], 1e-4)

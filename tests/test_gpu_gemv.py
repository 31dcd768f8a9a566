"""GPU parity of the GEMV family against the CPU oracle, through the C ABI.

Bar: activation codes, int32 block dots and dequantised weights bit-exact;
f32 outputs within 1e-5 x max|ref| (the reference's own tests measure
error against the output scale, e.g. quant.rs:1200-1206); matvec_many
bit-identical to single matvecs (quant.rs:1079-1108).
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

import kvad_amd as K  # noqa: E402  (fails loudly without libkvad_hip.so)

RTOL = 1e-5


def close(got, want, rtol=RTOL):
    scale = max(float(np.max(np.abs(want))), 1e-30)
    err = float(np.max(np.abs(got.astype(np.float64) - want)))
    assert err <= rtol * scale, f"max err {err:.3e} vs scale {scale:.3e}"


def say(*a):
    print("[case]", *a, flush=True)


def make(ctx, prec, rows, cols, seed, scale=0.02):
    w = O.normal(seed, rows * cols, scale)
    if prec == "q8":
        s, q = O.quantize_q8(w, rows, cols)
        return K.Weight.from_q8(ctx, rows, cols, s, q), (s, q)
    if prec == "q4":
        s, q = O.quantize_q4(w, rows, cols)
        return K.Weight.from_q4(ctx, rows, cols, s, q), (s, q)
    if prec == "q4k":
        b = O.quantize_q4k(w, rows, cols)
        return K.Weight.from_q4k(ctx, rows, cols, b), (b,)
    return K.Weight.from_f32(ctx, w.reshape(rows, cols)), (w,)


def oracle_matvec(prec, parts, rows, cols, x, bias=None):
    if prec == "q8":
        return O.matvec_q8(*parts, rows, cols, x, bias)
    if prec == "q4":
        return O.matvec_q4(*parts, rows, cols, x, bias)
    if prec == "q4k":
        return O.matvec_q4k(parts[0], rows, cols, x, bias)
    return O.matvec_f32(parts[0], rows, cols, x, bias)


def oracle_dots(prec, parts, rows, cols, x):
    xq, _, xsum = O.qact(x)
    if prec == "q8":
        return O.block_dots_q8(parts[1], rows, cols, xq)
    if prec == "q4":
        return O.block_dots_q4(parts[1], rows, cols, xq, xsum)
    return O.block_dots_q4k(parts[0], rows, cols, xq)


@pytest.mark.parametrize("n", [32, 896, 4864, 14336])
def test_activation_quantiser_is_bit_exact(ctx, n):
    say("qact", n)
    x = O.normal(7, n)
    x[:32] *= 1000.0  # an outlier block
    x[32:64] = 0.0    # an all-zero block
    x[64:96] *= 1e-38  # scales below the normal range: the divides' branch
    x[96:128] *= 1e-41  # subnormal inputs
    x[128:160] = np.float32(3e38) * np.sign(x[128:160])  # near the largest float
    qs, sc, su = K.qact(ctx, x)
    q2, s2, u2 = O.qact(x)
    np.testing.assert_array_equal(qs, q2)
    np.testing.assert_array_equal(sc.view(np.uint32), s2.view(np.uint32))
    np.testing.assert_array_equal(su, u2)


def test_quantiser_arithmetic_over_every_float(ctx):
    # the scale amax / 127, its inverse and the rounding of quant.rs:1052-1059
    # as the device computes them (a Markstein-corrected product and
    # reciprocal, an add-and-truncate rounding), against IEEE division and
    # round-half-away-from-zero for all 2^32 floats
    say("quantiser arithmetic, every float")
    assert K.quant_check(ctx) == (0, 0, 0)


SHAPES = {
    "q8": [(1, 32), (37, 64), (203, 96), (4864, 896), (896, 4864), (2048, 1408), (1408, 2816)],
    "q4": [(1, 32), (37, 64), (203, 96), (4864, 896), (896, 4864), (2048, 1408), (1408, 2816)],
    "q4k": [(1, 256), (37, 512), (64, 1024), (4096, 4096)],
    "f32": [(1, 3), (3, 2), (37, 64), (203, 97), (896, 896)],
}


@pytest.mark.parametrize("prec", ["q8", "q4", "q4k"])
def test_block_dots_are_bit_exact(ctx, prec):
    for rows, cols in SHAPES[prec]:
        say("dots", prec, rows, cols)
        w, parts = make(ctx, prec, rows, cols, seed=rows + cols)
        x = O.normal(rows * 7 + 1, cols)
        np.testing.assert_array_equal(w.block_dots(x), oracle_dots(prec, parts, rows, cols, x))


@pytest.mark.parametrize("prec", ["q8", "q4", "q4k", "f32"])
def test_dequantised_rows_are_bit_exact(ctx, prec):
    for rows, cols in SHAPES[prec][:4]:
        say("row", prec, rows, cols)
        w, parts = make(ctx, prec, rows, cols, seed=3 * rows + cols)
        for r in sorted({0, rows // 2, rows - 1}):
            got = w.row(r)
            if prec == "q8":
                want = O.row_q8(*parts, cols, r)
            elif prec == "q4":
                want = O.row_q4(*parts, cols, r)
            elif prec == "q4k":
                want = O.row_q4k(parts[0], cols, r)
            else:
                want = parts[0][r * cols:(r + 1) * cols]
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("prec", ["q8", "q4", "q4k", "f32"])
def test_matvec_matches_the_oracle(ctx, prec):
    for rows, cols in SHAPES[prec]:
        say("matvec", prec, rows, cols)
        w, parts = make(ctx, prec, rows, cols, seed=rows * 3 + cols)
        x = O.normal(rows + 11, cols)
        close(w.matvec_bt(x), oracle_matvec(prec, parts, rows, cols, x))
        bias = O.normal(rows + 12, rows)
        close(w.matvec_bt(x, bias), oracle_matvec(prec, parts, rows, cols, x, bias))


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (14336, 4096), (4096, 14336)])
def test_q4k_llama_shapes(ctx, rows, cols):
    say("q4k llama", rows, cols)
    w, parts = make(ctx, "q4k", rows, cols, seed=rows ^ cols)
    x = O.normal(cols, cols)
    close(w.matvec_bt(x), O.matvec_q4k(parts[0], rows, cols, x))
    np.testing.assert_array_equal(w.block_dots(x), oracle_dots("q4k", parts, rows, cols, x))


def test_matvec_is_deterministic(ctx):
    say("determinism")
    w, parts = make(ctx, "q4k", 4096, 4096, seed=5)
    x = O.normal(6, 4096)
    first = w.matvec_bt(x)
    for _ in range(5):
        np.testing.assert_array_equal(w.matvec_bt(x), first)


@pytest.mark.parametrize("prec", ["q8", "q4"])
def test_many_matvecs_at_once_equal_them_one_at_a_time(ctx, prec):
    # quant.rs:1079-1108, shapes and sharing as there
    say("matvec_many", prec)
    t = lambda r, c, s: O.normal(s, r * c, 0.1)
    x = O.normal(1, 64, 0.1)
    h = O.normal(2, 96, 0.1)
    ws = []
    for (r, c, s) in [(37, 64, 3), (5, 64, 4), (1, 96, 5), (203, 96, 6)]:
        w = t(r, c, s)
        if prec == "q8":
            sc, q = O.quantize_q8(w, r, c)
            ws.append(K.Weight.from_q8(ctx, r, c, sc, q))
        else:
            sc, q = O.quantize_q4(w, r, c)
            ws.append(K.Weight.from_q4(ctx, r, c, sc, q))
    jobs = [(ws[0], x), (ws[1], x), (ws[2], h), (ws[3], h)]
    many = K.matvec_many(ctx, jobs)
    assert many is not None
    for k, ((w, xx), got) in enumerate(zip(jobs, many)):
        np.testing.assert_array_equal(got, w.matvec_bt(xx), err_msg=f"job {k}")
    f = K.Weight.from_f32(ctx, t(4, 64, 7).reshape(4, 64))
    assert K.matvec_many(ctx, [(f, x)]) is None


def test_matvec_many_mixes_precisions_and_widths(ctx):
    say("matvec_many mixed")
    w1, p1 = make(ctx, "q8", 1408, 2048, 1)
    w2, p2 = make(ctx, "q4k", 1408, 2048, 2)
    w3, p3 = make(ctx, "q4", 2048, 1408, 3)
    x = O.normal(4, 2048)
    h = O.normal(5, 1408)
    ys = K.matvec_many(ctx, [(w1, x), (w2, x), (w3, h)])
    np.testing.assert_array_equal(ys[0], w1.matvec_bt(x))
    np.testing.assert_array_equal(ys[1], w2.matvec_bt(x))
    np.testing.assert_array_equal(ys[2], w3.matvec_bt(h))
    close(ys[1], O.matvec_q4k(p2[0], 1408, 2048, x))


def test_bad_shapes_are_errors_not_crashes(ctx):
    say("errors")
    with pytest.raises(K.KvadError):
        K.Weight.from_q8(ctx, 4, 33, np.zeros(4, np.float32), np.zeros(4 * 33, np.int8))
    with pytest.raises(K.KvadError):
        K.Weight.from_q4k(ctx, 4, 300, np.zeros(4 * 300, np.uint8))
    w, _ = make(ctx, "q8", 8, 64, 1)
    with pytest.raises(K.KvadError):
        w.row(8)


@pytest.mark.parametrize("prec", ["q8", "q4", "q4k"])
def test_device_quantiser_is_bit_exact(ctx, prec):
    # Weight::quantize (quant.rs:209-281) on the device vs the CPU quantiser
    rows, cols = (64, 1024) if prec == "q4k" else (96, 896)
    say("quantize", prec, rows, cols)
    w = O.normal(31, rows * cols, 0.02)
    w[:32] = 0.0          # an all-zero block
    w[40] = 3.0           # an outlier
    code = {"q8": K.Q8, "q4": K.Q4, "q4k": K.Q4K}[prec]
    dw = K.Weight.quantize(ctx, w.reshape(rows, cols), code)
    sc, qs = dw.parts()
    if prec == "q8":
        s2, q2 = O.quantize_q8(w, rows, cols)
    elif prec == "q4":
        s2, q2 = O.quantize_q4(w, rows, cols)
    else:
        s2, q2 = None, O.quantize_q4k(w, rows, cols)
    np.testing.assert_array_equal(qs, q2)
    if s2 is not None:
        np.testing.assert_array_equal(sc.view(np.uint32), s2.view(np.uint32))


def test_closing_a_context_frees_its_objects_first():
    # objects still alive when their context closes are freed with it (their
    # frees lock the context, so they may not outlive it); freeing them again
    # afterwards, or collecting them, does nothing
    say("context close with live objects")
    c = K.Context(0)
    w, _ = make(c, "q8", 64, 64, seed=1)
    kv = K.KvCache(c, 1, 64, 64, 4)
    c.close()
    assert w.h is None and kv.h is None and c.h is None
    w.free()
    kv.free()
    del w, kv

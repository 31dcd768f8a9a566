"""Pins the CPU oracle (oracle/kvad_oracle.c) before anything is checked
against it.

Each test is one of:
  * a known-answer or invariant test the reference itself holds, restated
    (file:line given), or
  * a check the mathematics fixes, written in a different form from the
    oracle's (integer brute force, float64 dequantise-then-dot, textbook
    softmax attention), chosen so a dropped term, swapped nibble or wrong
    index fails it.
No GPU; runs in seconds.
"""
import math

import numpy as np
import pytest

import oracle as O


def rust_xorshift_normal(seed: int, n: int) -> np.ndarray:
    """Independent restatement of nervus Rng (crates/nervus/src/rng.rs:7-39) in
    Python integers and float64 maths rounded to f32 at each step."""
    state = seed if seed else 0x9E3779B97F4A7C15
    mask = (1 << 64) - 1
    out = np.empty(n, np.float32)

    def nxt():
        nonlocal state
        x = state
        x ^= x >> 12
        x ^= (x << 25) & mask
        x ^= x >> 27
        state = x
        return (x * 0x2545F4914F6CDD1D) & mask

    def uni():
        return np.float32(nxt() >> 40) / np.float32(1 << 24)

    for i in range(n):
        u1 = max(uni(), np.float32(np.finfo(np.float32).tiny))
        u2 = uni()
        a = np.float32(-2.0) * np.float32(math.log(u1))
        b = np.float32(6.2831855) * u2
        out[i] = np.float32(math.sqrt(a)) * np.float32(math.cos(b))
    return out


def test_rng_matches_an_independent_xorshift_box_muller():
    got = O.normal(42, 2000)
    want = rust_xorshift_normal(42, 2000)
    # uniform draws are exact integer work; log/cos may differ by an ulp
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=2e-7)
    assert abs(float(np.mean(got))) < 0.1 and abs(float(np.std(got)) - 1.0) < 0.1
    # seed 0 is remapped, not a fixed point (rng.rs:13-16)
    z = O.normal(0, 4)
    assert np.all(np.isfinite(z)) and np.any(z != 0)


# ---------------------------------------------------------------------------
# quantisation (quant.rs:209-281, 1044-1066)
# ---------------------------------------------------------------------------

def round_half_away(t: np.ndarray) -> np.ndarray:
    t64 = t.astype(np.float64)
    return np.sign(t64) * np.floor(np.abs(t64) + 0.5)


def q8_numpy(w: np.ndarray):
    b = w.reshape(-1, 32).astype(np.float32)
    amax = np.max(np.abs(b), axis=1)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(scale > 0, np.float32(1.0) / scale, np.float32(0.0)).astype(np.float32)
    t = (b * inv[:, None]).astype(np.float32)
    q = np.clip(round_half_away(t), -127, 127).astype(np.int8)
    return scale, q.reshape(-1)


def test_q8_quantiser_matches_numpy_and_its_invariants():
    rows, cols = 16, 256
    w = O.normal(3, rows * cols, 0.1)
    s, q = O.quantize_q8(w, rows, cols)
    s2, q2 = q8_numpy(w)
    np.testing.assert_array_equal(s, s2)
    np.testing.assert_array_equal(q, q2)
    qb = q.reshape(-1, 32)
    # the extreme of every nonzero block lands on +-127
    assert np.all(np.max(np.abs(qb.astype(int)), axis=1) == 127)
    # reconstruction within half a step
    back = (qb.astype(np.float32) * s[:, None]).reshape(-1)
    assert np.all(np.abs(back - w) <= 0.5 * np.repeat(s, 32) * (1 + 1e-6) + 1e-12)


def round_trip_error(precision: str) -> float:
    # quant.rs:1110-1126: 8x256 ~ N(0, 0.1), relative RMS error via Weight::row
    t = O.normal(1, 8 * 256, 0.1)
    if precision == "q8":
        s, q = O.quantize_q8(t, 8, 256)
        back = np.concatenate([O.row_q8(s, q, 256, r) for r in range(8)])
    else:
        s, q = O.quantize_q4(t, 8, 256)
        back = np.concatenate([O.row_q4(s, q, 256, r) for r in range(8)])
    num = np.sum((back.astype(np.float64) - t) ** 2)
    den = np.sum(t.astype(np.float64) ** 2)
    return float(np.sqrt(num / den))


def test_quantisation_error_is_within_expectations():
    # quant.rs:1128-1138
    q8, q4 = round_trip_error("q8"), round_trip_error("q4")
    assert q8 < 0.01, q8
    assert q4 < 0.15, q4
    assert q8 < q4


def test_a_single_outlier_does_not_destroy_the_row():
    # quant.rs:1140-1159
    data = np.full(256, 0.01, np.float32)
    data[0] = 40.0
    s, q = O.quantize_q8(data, 1, 256)
    back = O.row_q8(s, q, 256, 0)
    assert abs(back[0] - 40.0) < 0.2
    assert abs(back[200] - 0.01) < 1e-4
    assert abs(back[5]) < 0.4


def test_exact_zero_stays_exact():
    # quant.rs:1161-1167
    s, q = O.quantize_q4(np.zeros(32, np.float32), 1, 32)
    assert np.all(O.row_q4(s, q, 32, 0) == 0.0)
    s, q = O.quantize_q8(np.zeros(32, np.float32), 1, 32)
    assert np.all(O.row_q8(s, q, 32, 0) == 0.0)


def test_storage_matches_the_advertised_bits_per_weight():
    # quant.rs:1210-1219
    n = 32 * 256
    t = O.normal(3, n, 0.1)
    s8, q8 = O.quantize_q8(t, 32, 256)
    s4, q4 = O.quantize_q4(t, 32, 256)
    assert s8.nbytes + q8.nbytes == n + n // 32 * 4
    assert s4.nbytes + q4.nbytes == n // 2 + n // 32 * 4
    assert O.quantize_q4k(t, 32, 256).nbytes == n // 256 * 144


def test_q4_codes_use_all_sixteen_levels_and_the_extreme_lands_on_minus_8():
    # quant.rs:234-255: the signed extreme maps onto code 0 (= -8)
    w = O.normal(9, 64 * 32, 0.05)
    s, q = O.quantize_q4(w, 64, 32)
    codes = np.stack([q & 0xF, q >> 4], axis=1)
    assert set(np.unique(codes)) == set(range(16))
    for b in range(64):
        blk = w[b * 32:(b + 1) * 32]
        e = int(np.argmax(np.abs(blk)))
        byte = q[b * 16 + (e % 16)]
        code = (byte & 0xF) if e < 16 else (byte >> 4)
        assert code == 0, (b, e, code)


def test_unpacking_a_nibble_row_gives_the_weights_it_encodes():
    # quant.rs:1254-1295 (the layout, checked on Weight::row): low nibble is
    # the first half of a block, high nibble the second half, bias 8
    rows, cols = 4, 96
    s, q = O.quantize_q4(O.normal(7, rows * cols, 0.1), rows, cols)
    for r in (2, 3):
        out = O.row_q4(s, q, cols, r)
        for b in range(cols // 32):
            sc = s[r * cols // 32 + b]
            for j in range(16):
                byte = int(q[r * cols // 2 + b * 16 + j])
                assert out[b * 32 + j] == np.float32((byte & 0xF) - 8) * sc
                assert out[b * 32 + 16 + j] == np.float32((byte >> 4) - 8) * sc


def test_qact_matches_the_weight_quantiser_and_sums_its_codes():
    x = O.normal(7, 4864)
    qs, sc, su = O.qact(x)
    s2, q2 = q8_numpy(x)
    np.testing.assert_array_equal(qs, q2)
    np.testing.assert_array_equal(sc, s2)
    np.testing.assert_array_equal(su, qs.reshape(-1, 32).astype(np.int32).sum(axis=1))


# ---------------------------------------------------------------------------
# block dots (quant.rs:168-189, 426-440; simd.rs:273-316)
# ---------------------------------------------------------------------------

def test_q8_block_dots_equal_integer_brute_force():
    rows, cols = 37, 896
    s, q = O.quantize_q8(O.normal(5, rows * cols, 0.02), rows, cols)
    xq, _, _ = O.qact(O.normal(6, cols))
    got = O.block_dots_q8(q, rows, cols, xq)
    want = (q.reshape(rows, -1, 32).astype(np.int64) * xq.reshape(1, -1, 32)).sum(axis=2)
    np.testing.assert_array_equal(got, want)


def test_the_nibble_kernel_matches_longhand():
    # simd.rs:273-316: nine blocks, every nibble value, activations -125..125;
    # the unsigned-minus-8*sum form against signed codes written out
    blocks = 9
    packed = np.array([(i * 37 + 11) & 0xFF for i in range(blocks * 16)], np.uint8)
    acts = np.array([((i * 13) % 251) - 125 for i in range(blocks * 32)], np.int8)
    assert acts.min() == -125 and acts.max() == 125
    assert len({int(b) & 0xF for b in packed} | {int(b) >> 4 for b in packed}) == 16
    sums = acts.reshape(-1, 32).astype(np.int32).sum(axis=1)
    got = O.block_dots_q4(packed, 1, blocks * 32, acts, sums)[0]
    want = []
    for b in range(blocks):
        d = 0
        for j in range(16):
            byte = int(packed[b * 16 + j])
            d += ((byte & 0xF) - 8) * int(acts[b * 32 + j])
            d += ((byte >> 4) - 8) * int(acts[b * 32 + 16 + j])
        want.append(d)
    np.testing.assert_array_equal(got, want)


# ---------------------------------------------------------------------------
# GEMV (quant.rs:410-512) against float64 dequantise-then-dot
# ---------------------------------------------------------------------------

def deq_dot_f64(wrows: np.ndarray, x: np.ndarray) -> np.ndarray:
    """sum_k wdeq[k] * xdeq[k] in float64, the exact value of the two-pass form."""
    xq, xs, _ = O.qact(x)
    xd = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 32)
    return wrows.astype(np.float64) @ xd


@pytest.mark.parametrize("rows,cols", [(96, 64), (4864, 896), (896, 4864)])
def test_q8_matvec_equals_the_exact_two_pass_value(rows, cols):
    w = O.normal(42, rows * cols, 0.02)
    x = O.normal(7, cols)
    s, q = O.quantize_q8(w, rows, cols)
    wd = q.reshape(rows, cols).astype(np.float64) * np.repeat(s.astype(np.float64), 32).reshape(rows, cols)
    y = O.matvec_q8(s, q, rows, cols, x)
    want = deq_dot_f64(wd, x)
    assert np.max(np.abs(y - want)) <= 1e-6 * np.max(np.abs(want))


def test_q4_matvec_equals_the_exact_two_pass_value():
    rows, cols = 203, 96
    w = O.normal(6, rows * cols, 0.1)
    x = O.normal(2, cols)
    s, q = O.quantize_q4(w, rows, cols)
    wd = np.stack([O.row_q4(s, q, cols, r) for r in range(rows)]).astype(np.float64)
    y = O.matvec_q4(s, q, rows, cols, x)
    want = deq_dot_f64(wd, x)
    assert np.max(np.abs(y - want)) <= 1e-6 * np.max(np.abs(want))


def test_quantised_matvec_bt_agrees_with_f32():
    # quant.rs:1189-1208
    t = O.normal(11, 96 * 64, 0.1)
    x = O.normal(5, 64)
    ref = O.matvec_f32(t, 96, 64, x)
    scale = np.max(np.abs(ref))
    s8, q8 = O.quantize_q8(t, 96, 64)
    s4, q4 = O.quantize_q4(t, 96, 64)
    assert np.max(np.abs(O.matvec_q8(s8, q8, 96, 64, x) - ref)) <= 0.03 * scale
    assert np.max(np.abs(O.matvec_q4(s4, q4, 96, 64, x) - ref)) <= 0.35 * scale


def test_bias_is_applied_in_every_precision():
    # quant.rs:1169-1187
    t = O.normal(7, 16 * 64, 0.1)
    x = O.normal(99, 64)
    bias = O.normal(98, 16)
    for name in ("f32", "q8", "q4"):
        if name == "f32":
            f = lambda b: O.matvec_f32(t, 16, 64, x, b)
        elif name == "q8":
            s, q = O.quantize_q8(t, 16, 64)
            f = lambda b: O.matvec_q8(s, q, 16, 64, x, b)
        else:
            s, q = O.quantize_q4(t, 16, 64)
            f = lambda b: O.matvec_q4(s, q, 16, 64, x, b)
        assert np.max(np.abs(f(bias) - (f(None) + bias))) < 1e-4, name


def test_matvec_bt_matches_hand_computation():
    # tensor.rs:535-540 and 527-533
    w = np.array([[1, 0], [0, 1], [1, 1]], np.float32)
    assert list(O.matvec_f32(w, 3, 2, np.array([3, 5], np.float32))) == [3.0, 5.0, 8.0]
    wt = np.array([[1, 2, 3], [4, 5, 6]], np.float32).T.copy()
    assert list(O.matvec_f32(wt, 3, 2, np.array([1, 2], np.float32))) == [9.0, 12.0, 15.0]


def test_dequant_baseline_equals_its_float64_value():
    # quant.rs:522-589: activations stay f32
    rows, cols = 64, 256
    w = O.normal(4, rows * cols, 0.05)
    x = O.normal(8, cols)
    s8, q8 = O.quantize_q8(w, rows, cols)
    wd = np.stack([O.row_q8(s8, q8, cols, r) for r in range(rows)]).astype(np.float64)
    y = O.matvec_dequant(1, s8, q8, rows, cols, x)
    want = wd @ x.astype(np.float64)
    assert np.max(np.abs(y - want)) <= 1e-5 * np.max(np.abs(want))
    s4, q4 = O.quantize_q4(w, rows, cols)
    wd = np.stack([O.row_q4(s4, q4, cols, r) for r in range(rows)]).astype(np.float64)
    y = O.matvec_dequant(2, s4, q4, rows, cols, x)
    want = wd @ x.astype(np.float64)
    assert np.max(np.abs(y - want)) <= 1e-5 * np.max(np.abs(want))


# ---------------------------------------------------------------------------
# batched prefill (quant.rs:751-907; tensor.rs:102-186)
# ---------------------------------------------------------------------------

def ref_lcg(n: int, seed=0x12345678):
    # tensor.rs:492-498: the reference test's own xorshift
    out = np.empty(n, np.float32)
    mask = (1 << 64) - 1
    for i in range(n):
        seed ^= (seed << 13) & mask
        seed ^= seed >> 7
        seed ^= (seed << 17) & mask
        out[i] = np.float32(seed >> 40) / np.float32(8388608.0) - np.float32(1.0)
    return out, seed


def test_gemm_matches_running_the_rows_one_at_a_time():
    # tensor.rs:487-516
    for rows, cols, m in [(9, 13, 7), (8, 16, 4), (5, 32, 1), (6, 8, 9)]:
        w, seed = ref_lcg(rows * cols)
        xs, _ = ref_lcg(m * cols, seed)
        out_t = O.gemm_f32(xs, m, w, rows, cols)
        for i in range(m):
            single = O.matvec_f32(w, rows, cols, xs[i * cols:(i + 1) * cols])
            for r in range(rows):
                assert abs(single[r] - out_t[r * m + i]) < 1e-5


def test_gemm_equals_float64():
    rows, cols, m = 70, 100, 11
    w = O.normal(1, rows * cols)
    xs = O.normal(2, m * cols)
    out_t = O.gemm_f32(xs, m, w, rows, cols).reshape(rows, m)
    want = w.reshape(rows, cols).astype(np.float64) @ xs.reshape(m, cols).astype(np.float64).T
    assert np.max(np.abs(out_t - want)) < 1e-4 * np.max(np.abs(want))


def test_batched_matmul_agrees_with_row_by_row():
    # quant.rs:1304-1329 with the x86 path: every element equals the single
    # matvec to the bit (row_dot and qrow are the same two passes)
    t = O.normal(5, 70 * 128, 0.1)
    for m in (1, 2, 5):
        xs = O.normal(4242 + m, m * 128)
        s8, q8 = O.quantize_q8(t, 70, 128)
        s4, q4 = O.quantize_q4(t, 70, 128)
        b8 = O.matmul_q8(s8, q8, 70, 128, xs, m).reshape(m, 70)
        b4 = O.matmul_q4(s4, q4, 70, 128, xs, m).reshape(m, 70)
        bf = O.matmul_f32(t, 70, 128, xs, m).reshape(m, 70)
        for i in range(m):
            x = xs[i * 128:(i + 1) * 128]
            np.testing.assert_array_equal(b8[i], O.matvec_q8(s8, q8, 70, 128, x))
            np.testing.assert_array_equal(b4[i], O.matvec_q4(s4, q4, 70, 128, x))
            single = O.matvec_f32(t, 70, 128, x)
            assert np.max(np.abs(bf[i] - single)) <= 1e-4 * max(np.max(np.abs(single)), 1e-3)


# ---------------------------------------------------------------------------
# Q4_K (gpu/src/mpp.rs:241-315)
# ---------------------------------------------------------------------------

def pack_scale_min_ggml(sc, m) -> np.ndarray:
    """GGML's k-quant scale packing as mpp.rs:273-275 describes it: the first
    four scales and mins whole in the low six bits of bytes 0-3 and 4-7, the
    last four as nibbles of bytes 8-11 topped up with the spare two bits of
    bytes 0-7."""
    q = np.zeros(12, np.uint8)
    for j in range(4):
        q[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4)
    return q


def test_q4k_codec_round_trips_scales_and_codes():
    rows, cols = 8, 512
    w = O.normal(13, rows * cols, 0.02)
    blocks = O.quantize_q4k(w, rows, cols).reshape(-1, 144)
    rng = np.random.default_rng(0)
    for blk in blocks:
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        q = pack_scale_min_ggml(sc, mn)
        # the decoder in the oracle and the GPU reads q this way (mpp.rs:276-282)
        for j in range(8):
            if j < 4:
                a, b = q[j] & 63, q[j + 4] & 63
            else:
                a = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4)
                b = (q[j + 4] >> 4) | ((q[j] >> 6) << 4)
            assert (a, b) == (sc[j], mn[j])
        break
    # dequantised rows reproduce the weights to quantisation accuracy
    back = np.concatenate([O.row_q4k(blocks, cols, r) for r in range(rows)])
    rel = np.sqrt(np.sum((back.astype(np.float64) - w) ** 2) / np.sum(w.astype(np.float64) ** 2))
    assert rel < 0.12, rel


def q4k_decode_numpy(blocks: np.ndarray, rows: int, cols: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """codes[rows, cols] (0..15), dl[rows, cols/32], ml[rows, cols/32] read
    straight from the block bytes, written independently of the oracle."""
    nsb = cols // 256
    b = blocks.reshape(rows, nsb, 144)
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float32)[..., 0]
    dmin = b[:, :, 2:4].copy().view(np.float16).astype(np.float32)[..., 0]
    s = b[:, :, 4:16].astype(np.int32)
    sc = np.zeros((rows, nsb, 8), np.int32)
    mn = np.zeros((rows, nsb, 8), np.int32)
    sc[..., :4] = s[..., 0:4] & 63
    mn[..., :4] = s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 0xF) | ((s[..., 0:4] >> 6) << 4)
    mn[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    qs = b[:, :, 16:].astype(np.int32).reshape(rows, nsb, 4, 32)
    codes = np.zeros((rows, nsb, 8, 32), np.int32)
    codes[:, :, 0::2, :] = qs & 0xF
    codes[:, :, 1::2, :] = qs >> 4
    dl = (d[..., None] * sc.astype(np.float32)).astype(np.float32)
    ml = (dmin[..., None] * mn.astype(np.float32)).astype(np.float32)
    return codes.reshape(rows, cols), dl.reshape(rows, -1), ml.reshape(rows, -1)


def test_q4k_rows_equal_an_independent_decoder():
    rows, cols = 6, 768
    blocks = O.quantize_q4k(O.normal(21, rows * cols, 0.02), rows, cols)
    codes, dl, ml = q4k_decode_numpy(blocks, rows, cols)
    want = (np.repeat(dl, 32, axis=1) * codes.astype(np.float32)).astype(np.float32) - np.repeat(ml, 32, axis=1)
    got = np.stack([O.row_q4k(blocks, cols, r) for r in range(rows)])
    np.testing.assert_array_equal(got, want.astype(np.float32))


def test_q4k_block_dots_and_gemv_equal_the_exact_value():
    rows, cols = 64, 1024
    blocks = O.quantize_q4k(O.normal(22, rows * cols, 0.02), rows, cols)
    x = O.normal(23, cols)
    xq, xs, xsum = O.qact(x)
    codes, dl, ml = q4k_decode_numpy(blocks, rows, cols)
    dots = O.block_dots_q4k(blocks, rows, cols, xq)
    want = (codes.reshape(rows, -1, 32).astype(np.int64) * xq.reshape(1, -1, 32)).sum(axis=2)
    np.testing.assert_array_equal(dots, want)
    # y = sum_k (dl*q - ml)[k] * xs*xq[k], exactly, in float64
    wd = np.repeat(dl.astype(np.float64), 32, axis=1) * codes - np.repeat(ml.astype(np.float64), 32, axis=1)
    ywant = deq_dot_f64(wd, x)
    y = O.matvec_q4k(blocks, rows, cols, x)
    assert np.max(np.abs(y - ywant)) <= 1e-6 * np.max(np.abs(ywant))


def test_q4k_cpu_baseline_loop_equals_the_oracle_to_the_bit():
    # the CPU baseline's loop (scales decoded once per sub-block) computes the
    # oracle's integers and pass-2 steps; at several widths and thread counts
    for rows, cols in [(1, 256), (37, 512), (64, 4096), (5, 14336)]:
        blocks = O.quantize_q4k(O.normal(30 + rows, rows * cols, 0.02), rows, cols)
        x = O.normal(31 + cols, cols)
        x[:32] *= 500.0
        bias = O.normal(32, rows)
        want = O.matvec_q4k(blocks, rows, cols, x, bias)
        np.testing.assert_array_equal(O.matvec_q4k_fast(blocks, rows, cols, x, bias), want)
        old = O.threads()
        try:
            O.set_threads(1)
            np.testing.assert_array_equal(O.matvec_q4k_fast(blocks, rows, cols, x, bias), want)
        finally:
            O.set_threads(old)


def test_f16_conversion_round_trips_and_rounds_to_nearest_even():
    for v in [0.0, 1.0, -2.5, 65504.0, 6.1035156e-05, 5.9604645e-08, 1e-3, 0.333]:
        h = O.f32_to_f16(v)
        assert np.float16(v).view(np.uint16) == h, v
        assert O.f16_to_f32(h) == float(np.float16(v))
    vals = O.normal(77, 5000, 3.0)
    hs = np.array([O.f32_to_f16(float(v)) for v in vals], np.uint16)
    np.testing.assert_array_equal(hs, vals.astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------------------
# small f32 pieces (tensor.rs)
# ---------------------------------------------------------------------------

def test_softmax_sums_to_one_and_survives_large_inputs():
    # tensor.rs:554-564
    x = O.softmax(np.array([1000.0, 1000.0, 1000.0], np.float32))
    assert np.all(np.abs(x - 1.0 / 3.0) < 1e-6)
    y = O.softmax(np.array([0.0, 1.0, 2.0], np.float32))
    assert abs(float(y.sum()) - 1.0) < 1e-6 and y[2] > y[1] > y[0]


def test_dot_is_the_float64_dot_to_rounding():
    for n in (1, 7, 8, 64, 100):
        a, b = O.normal(1, n), O.normal(2, n)
        want = float(a.astype(np.float64) @ b.astype(np.float64))
        assert abs(O.dot(a, b) - want) <= 1e-5 * max(1.0, float(np.sum(np.abs(a * b))))


def test_rms_norm_rescales_without_centring():
    # tensor.rs:583-597
    y = O.rms_norm(np.ones(8, np.float32), np.ones(8, np.float32), 1e-6)
    assert np.all(np.abs(y - 1.0) < 1e-4)
    y = O.rms_norm(np.array([3.0, -4.0, 0.0, 5.0], np.float32), np.ones(4, np.float32), 1e-6)
    assert abs(math.sqrt(float(np.mean(y.astype(np.float64) ** 2))) - 1.0) < 1e-4


def test_swiglu_gates():
    # tensor.rs:599-610
    g = O.swiglu(np.array([0.0, 10.0, -10.0], np.float32), np.array([2.0, 2.0, 2.0], np.float32))
    assert abs(g[0]) < 1e-6 and abs(g[1] - 20.0) < 0.01 and abs(g[2]) < 0.01


def test_rope_preserves_length_and_encodes_relative_position():
    # tensor.rs:612-650
    c, s = O.rope_tables(8, 64, 10000.0)
    x = np.array([1.0, 2.0, -1.0, 0.5, 3.0, -2.0, 0.25, 1.5], np.float32)
    y = O.rope_apply(c, s, 4, x, 37)
    assert abs(float(np.sum(x * x)) - float(np.sum(y * y))) < 1e-3
    assert np.all(np.abs(O.rope_apply(c, s, 4, x, 0) - x) < 1e-6)
    q = np.array([0.3, -1.2, 0.7, 2.0, -0.5, 1.1, 0.9, -0.4], np.float32)
    k = np.array([1.0, 0.4, -0.8, 0.2, 1.7, -1.3, 0.6, 0.1], np.float32)
    dot_at = lambda qp, kp: float(np.sum(O.rope_apply(c, s, 4, q, qp) * O.rope_apply(c, s, 4, k, kp)))
    ref = dot_at(10, 0)
    for start in (5, 20, 40, 50):
        assert abs(dot_at(start + 10, start) - ref) < 1e-3


# ---------------------------------------------------------------------------
# attention (model/mod.rs:769-819)
# ---------------------------------------------------------------------------

def attend_f64(n_head, n_kv, hd, q, k, v, L):
    kv_dim = n_kv * hd
    g = n_head // n_kv
    out = np.zeros((n_head, hd))
    K = k[:L * kv_dim].reshape(L, n_kv, hd).astype(np.float64)
    V = v[:L * kv_dim].reshape(L, n_kv, hd).astype(np.float64)
    for h in range(n_head):
        s = K[:, h // g, :] @ q[h * hd:(h + 1) * hd].astype(np.float64) / math.sqrt(hd)
        w = np.exp(s - s.max())
        w /= w.sum()
        out[h] = w @ V[:, h // g, :]
    return out.reshape(-1)


@pytest.mark.parametrize("n_head,n_kv,hd,L", [(14, 2, 64, 1), (14, 2, 64, 300), (32, 8, 128, 64), (4, 4, 16, 9)])
def test_attend_is_textbook_attention(n_head, n_kv, hd, L):
    kv_dim = n_kv * hd
    q = O.normal(1, n_head * hd)
    k = O.normal(2, L * kv_dim)
    v = O.normal(3, L * kv_dim)
    got = O.attend(n_head, n_kv, hd, q, k, v, L)
    want = attend_f64(n_head, n_kv, hd, q, k, v, L)
    assert np.max(np.abs(got - want)) <= 1e-5 * max(np.max(np.abs(want)), 1e-3)


def test_attend_at_one_position_returns_the_value_exactly():
    # w = 1 at L = 1, so each head's output is its KV head's value
    q, k, v = O.normal(4, 14 * 64), O.normal(5, 128), O.normal(6, 128)
    out = O.attend(14, 2, 64, q, k, v, 1).reshape(14, 64)
    for h in range(14):
        np.testing.assert_array_equal(out[h], v[(h // 7) * 64:(h // 7 + 1) * 64])


def test_attend_skips_weights_below_1e8():
    # mod.rs:807: one overwhelming key; the rest fall below 1e-8 and their
    # (huge) values must not leak in
    hd, L = 16, 5
    q = np.zeros(hd, np.float32)
    q[0] = 10.0
    k = np.zeros(L * hd, np.float32)
    k[0] = 40.0  # score 100 for position 0; the others score 0
    v = np.full(L * hd, 1e6, np.float32)
    v[:hd] = 1.0
    out = O.attend(1, 1, hd, q, k, v, L)
    np.testing.assert_array_equal(out, np.ones(hd, np.float32))


# ---------------------------------------------------------------------------
# router (model/ffn.rs:256-309)
# ---------------------------------------------------------------------------

def test_qwen3s_chosen_weights_are_renormalised_to_sum_to_one():
    # ffn.rs:1121-1147
    logits = np.array([0.0, 3.0, 1.0, -1.0, 2.0, 0.5, -2.0, 4.0], np.float32)
    picks = O.route(logits, 4, norm_topk=True)
    assert [e for e, _ in picks] == [7, 1, 4, 2]
    assert abs(sum(w for _, w in picks) - 1.0) < 1e-6
    assert abs(picks[0][1] / picks[1][1] - math.e) < 1e-5


def test_without_normalisation_the_weights_are_the_softmaxs_own():
    # ffn.rs:1149-1168
    logits = np.array([0.0, 3.0, 1.0, -1.0, 2.0, 0.5, -2.0, 4.0], np.float32)
    sm = O.softmax(logits)
    for e, w in O.route(logits, 4):
        assert abs(w - sm[e]) < 1e-6


def test_route_ties_pick_the_first_index():
    picks = O.route(np.array([1.0, 2.0, 2.0, 0.0], np.float32), 2)
    assert [e for e, _ in picks] == [1, 2]


def _moe_weights(hidden, inter, n_exp, seed, sh_inter=0):
    q = lambda s, r, c, sc: O.quantize_q8(O.normal(s, r * c, sc), r, c)
    router = q(seed, n_exp, hidden, 0.5)
    gate = q(seed + 1, n_exp * inter, hidden, 0.05)
    up = q(seed + 2, n_exp * inter, hidden, 0.05)
    down = q(seed + 3, n_exp * hidden, inter, 0.05)
    shared = None
    if sh_inter:
        shared = (q(seed + 4, sh_inter, hidden, 0.05), q(seed + 5, sh_inter, hidden, 0.05),
                  q(seed + 6, hidden, sh_inter, 0.05), sh_inter)
    return router, gate, up, down, shared


def test_moe_tokens_together_equal_tokens_alone():
    # prefill (grouped by expert, matmul_bt) against decode (matvec), bit for
    # bit: matmul_bt's x86 row_dot is the same arithmetic as matvec's qrow
    # (quant.rs:410-452, 865-907), and the mix adds in expert order either way
    hidden, inter, n_exp, k, m = 64, 32, 8, 3, 5
    r, g, u, d, sh = _moe_weights(hidden, inter, n_exp, 60, sh_inter=64)
    hs = O.normal(70, m * hidden)
    together = O.moe_run_q8(hs, m, hidden, inter, n_exp, k, r, g, u, d, sh).reshape(m, hidden)
    for i in range(m):
        alone = O.moe_run_q8(hs[i * hidden:(i + 1) * hidden], 1, hidden, inter, n_exp, k, r, g, u, d, sh)
        np.testing.assert_array_equal(together[i], alone)


def test_moe_is_the_weighted_sum_of_the_chosen_experts():
    # y = shared(x) + sum_x w_x ffn_x(x) over the router's picks, in float64
    # from the dequantised weights and the quantised activations
    hidden, inter, n_exp, k = 64, 32, 8, 3
    r, g, u, d, sh = _moe_weights(hidden, inter, n_exp, 80, sh_inter=32)
    x = O.normal(90, hidden)
    got = O.moe_run_q8(x, 1, hidden, inter, n_exp, k, r, g, u, d, sh)

    def deq(sq, rows, cols):
        s, q = sq
        return (q.reshape(rows, cols).astype(np.float64) * np.repeat(s.reshape(rows, cols // 32), 32, axis=1))

    def qx(v):
        q, s, _ = O.qact(v.astype(np.float32))
        return q.astype(np.float64) * np.repeat(s.astype(np.float64), 32)

    def ffn(G, U, D, width, v):
        a = qx(v)
        gg, uu = G @ a, U @ a
        h = gg / (1.0 + np.exp(-gg)) * uu
        return D @ qx(h)

    logits = deq(r, n_exp, hidden) @ qx(x)
    picks = O.route(logits.astype(np.float32), k)
    want = ffn(deq(sh[0], 32, hidden), deq(sh[1], 32, hidden), deq(sh[2], hidden, 32), 32, x)
    Gs, Us, Ds = deq(g, n_exp * inter, hidden), deq(u, n_exp * inter, hidden), deq(d, n_exp * hidden, inter)
    for e, w in sorted(picks):
        want = want + w * ffn(Gs[e * inter:(e + 1) * inter], Us[e * inter:(e + 1) * inter],
                              Ds[e * hidden:(e + 1) * hidden], inter, x)
    scale = float(np.max(np.abs(want)))
    # rounding only (measured 2e-7); a code of h landing on the other side of
    # a rounding boundary between the two paths would show as ~1e-3
    assert float(np.max(np.abs(got - want))) <= 1e-4 * scale


def test_interleaved_rope_is_the_half_split_rope_a_permutation_apart():
    # tensor.rs:430-436: the two conventions differ by a permutation of the
    # coordinates, applied to the vector before and undone after
    hd = 64
    c, s = O.rope_tables(hd, 20, 1e6)
    x = O.normal(3, hd)
    perm = np.r_[0:hd:2, 1:hd:2]  # interleaved pair (2i, 2i+1) -> (i, i + half)
    for pos in (0, 1, 7, 19):
        inter = O.rope_apply_interleaved(c, s, hd // 2, x, pos)
        split = O.rope_apply(c, s, hd // 2, x[perm], pos)
        np.testing.assert_array_equal(inter[perm], split)


# ---- latent attention (model/deepseek.rs:553-591) --------------------------

def _mla_f64(ql, qp, c, pe, scale):
    """Textbook softmax attention in float64 with the reference's skip of weights below 1e-8."""
    s = (ql.astype(np.float64) @ c.T.astype(np.float64) + qp.astype(np.float64) @ pe.T.astype(np.float64)) * scale
    w = np.exp(s - s.max(1, keepdims=True))
    w /= w.sum(1, keepdims=True)
    w[w < 1e-8] = 0.0
    return w @ c.astype(np.float64)


@pytest.mark.parametrize("H, L", [(16, 1), (16, 9), (5, 300)])
def test_mla_oracle_is_softmax_attention_over_the_latent(H, L):
    rng = np.random.default_rng(H * 1000 + L)
    ql, qp = rng.standard_normal((H, 512)).astype(np.float32), rng.standard_normal((H, 64)).astype(np.float32)
    c, pe = rng.standard_normal((L, 512)).astype(np.float32), rng.standard_normal((L, 64)).astype(np.float32)
    scale = 1.0 / np.sqrt(192.0)
    got = O.mla_attend(H, 512, 64, ql, qp, c, pe, L, scale).reshape(H, 512)
    want = _mla_f64(ql, qp, c, pe, scale)
    assert np.max(np.abs(got - want)) <= 2e-6 * np.max(np.abs(want))
    if L == 1:  # one position: every head's weight is 1, the latent comes back as it is
        assert np.array_equal(got, np.broadcast_to(c[0], (H, 512)))


def test_mla_oracle_drops_weights_below_1e_8():
    rng = np.random.default_rng(5)
    H, L = 2, 40
    ql, qp = rng.standard_normal((H, 512)).astype(np.float32), np.zeros((H, 64), np.float32)
    c, pe = rng.standard_normal((L, 512)).astype(np.float32), np.zeros((L, 64), np.float32)
    c[7] = -ql[0] * 3.0  # head 0 scores position 7 far below the rest
    scale = 1.0 / np.sqrt(192.0)
    got = O.mla_attend(H, 512, 64, ql, qp, c, pe, L, scale).reshape(H, 512)
    want = _mla_f64(ql, qp, c, pe, scale)
    assert np.max(np.abs(got - want)) <= 2e-6 * np.max(np.abs(want))
    s = (ql[0].astype(np.float64) @ c.T.astype(np.float64)) * scale
    w = np.exp(s - s.max()) / np.exp(s - s.max()).sum()
    assert w[7] < 1e-8 < w.max()  # the skip does apply here


# ---- the decoder's composition (O.Llm.forward) against a float64 restatement


def _f64_llm(spec, layers, embed, final, head, cos_t, sin_t, tokens):
    """The forward of llama.rs:224-289 between the embedding and the head
    (:384-415), restated in float64 numpy from dequantised q8 weights.  Each
    projection's input is quantised by the oracle's QActivation::new (the
    reference quantises there too); everything else -- norms, RoPE, the
    cache, attention with its 1e-8 skip (mod.rs:807), SwiGLU, the residual
    adds -- is computed here in float64, independently of the oracle's C."""
    e, hd, nh, nkv, eps = spec["n_embd"], spec["head_dim"], spec["n_head"], spec["n_kv_head"], spec["eps"]
    half, group = hd // 2, nh // nkv
    deq = lambda w, rows, cols: (np.repeat(np.asarray(w[0], np.float64).reshape(rows, cols // 32), 32, axis=1)
                                 * np.asarray(w[1], np.float64).reshape(rows, cols))

    def proj(w, rows, cols, x, bias=None):
        xq, xs, _ = O.qact(np.asarray(x, np.float32))
        y = deq(w, rows, cols) @ (np.repeat(np.asarray(xs, np.float64), 32) * xq)
        return y if bias is None else y + np.asarray(bias, np.float64)

    def norm(x, w):
        x = np.asarray(x, np.float64)
        return x / np.sqrt(np.mean(x * x) + eps) * np.asarray(w, np.float64)

    def rope(x, pos):
        c = np.asarray(cos_t, np.float64).reshape(-1, half)[pos]
        s = np.asarray(sin_t, np.float64).reshape(-1, half)[pos]
        if spec.get("rope_interleaved"):
            a, b = x[0::2].copy(), x[1::2].copy()
            x[0::2], x[1::2] = a * c - b * s, b * c + a * s
        else:
            a, b = x[:half].copy(), x[half:].copy()
            x[:half], x[half:] = a * c - b * s, b * c + a * s
        return x

    qd, kvd = nh * hd, nkv * hd
    kc = [[] for _ in layers]
    vc = [[] for _ in layers]
    out = []
    for pos, tok in enumerate(tokens):
        x = deq(embed, spec["vocab"], e)[tok]
        for l, L in enumerate(layers):
            h = norm(x, L["attn_norm"])
            q = proj(L["q"], qd, e, h, L.get("q_b"))
            k = proj(L["k"], kvd, e, h, L.get("k_b"))
            v = proj(L["v"], kvd, e, h, L.get("v_b"))
            for i in range(nh):
                q[i * hd:(i + 1) * hd] = rope(q[i * hd:(i + 1) * hd], pos)
            for i in range(nkv):
                k[i * hd:(i + 1) * hd] = rope(k[i * hd:(i + 1) * hd], pos)
            kc[l].append(k)
            vc[l].append(v)
            K_, V_ = np.array(kc[l]), np.array(vc[l])
            att = np.zeros(qd)
            for i in range(nh):
                j = (i // group) * hd
                sc = K_[:, j:j + hd] @ q[i * hd:(i + 1) * hd] / math.sqrt(hd)
                w = np.exp(sc - sc.max())
                w /= w.sum()
                w[w < 1e-8] = 0.0
                att[i * hd:(i + 1) * hd] = w @ V_[:, j:j + hd]
            x = x + proj(L["o"], e, qd, att)
            h = norm(x, L["mlp_norm"])
            g = proj(L["gate"], spec["n_ff"], e, h)
            u = proj(L["up"], spec["n_ff"], e, h)
            x = x + proj(L["down"], e, spec["n_ff"], g / (1.0 + np.exp(-g)) * u)
        out.append(proj(head, spec["vocab"], e, norm(x, final)))
    return out


def _two_layer_model(interleaved, seed=4000):
    # a 2-layer q8 model with Qwen2-style biases; layer weights N(0, 0.1) and
    # embeddings N(0, 0.05), so that every branch moves the logits by O(1)
    rng = iter(range(seed, seed + 1000))
    spec = dict(n_layer=2, n_embd=128, n_head=4, n_kv_head=2, head_dim=32, n_ff=256, vocab=64, n_ctx=16, eps=1e-6,
                rope_interleaved=int(interleaved))
    qd, kvd, e = 128, 64, 128
    q8 = lambda r, c, sc=0.1: O.quantize_q8(O.normal(next(rng), r * c, sc), r, c)
    vec = lambda n, b=1.0: (b + O.normal(next(rng), n, 0.1)).astype(np.float32)
    layers = []
    for _ in range(2):
        L = {n: q8(r, c) for n, (r, c) in dict(q=(qd, e), k=(kvd, e), v=(kvd, e), o=(e, qd), gate=(256, e),
                                                up=(256, e), down=(e, 256)).items()}
        L.update(attn_norm=vec(e), mlp_norm=vec(e), q_b=vec(qd, 0.0), k_b=vec(kvd, 0.0), v_b=vec(kvd, 0.0))
        layers.append(L)
    embed, final = q8(64, e, 0.05), vec(e)
    cos_t, sin_t = O.rope_tables(32, 16, 1e6)
    return spec, layers, embed, final, cos_t, sin_t


TOKENS = [3, 17, 60, 42, 7, 7, 1]


def _rel_errs(spec, layers, embed, final, cos_t, sin_t, oracle_layers=None):
    want = _f64_llm(spec, layers, embed, final, embed, cos_t, sin_t, TOKENS)
    ref = O.Llm(spec, oracle_layers or layers, embed, final, None, cos_t, sin_t)
    return [float(np.max(np.abs(ref.forward(t).astype(np.float64) - want[i]))) / float(np.max(np.abs(want[i])))
            for i, t in enumerate(TOKENS)]


@pytest.mark.parametrize("interleaved", [False, True])
def test_the_oracles_decoder_is_the_float64_composition(interleaved):
    # The oracle's logits agree with the float64 restatement to 1e-5 x max at
    # every step (measured: under 3e-7 -- f32 rounding in the norms,
    # attention and adds; no activation code moves across a boundary here).
    errs = _rel_errs(*_two_layer_model(interleaved))
    assert max(errs) <= 1e-5, errs


@pytest.mark.parametrize("slip", ["down", "o", "attn_norm", "v_b"])
def test_the_float64_composition_catches_a_wiring_slip(slip):
    # the same check against an oracle whose second layer has one part
    # planted wrong (its down / o projection zeroed, its attention norm
    # weights all one, its v bias dropped) fails by far more than the bar
    spec, layers, embed, final, cos_t, sin_t = _two_layer_model(False)
    L = dict(layers[1])
    if slip in ("down", "o"):
        L[slip] = (np.zeros_like(L[slip][0]), L[slip][1])
    elif slip == "attn_norm":
        L[slip] = np.ones_like(L[slip])
    else:
        L[slip] = np.zeros_like(L[slip])
    errs = _rel_errs(spec, layers, embed, final, cos_t, sin_t, oracle_layers=[layers[0], L])
    assert max(errs) > 1e-2, errs


# ---- a prompt's pass (O.Llm.forward_rows, Rows::Following) -----------------


def test_a_pass_of_rows_is_its_tokens_one_at_a_time_to_the_bit():
    # On x86 Weight::matmul_bt runs row_dot, the same two passes as qrow, per
    # (row, token) (quant.rs:751-907; the SMMLA pair path is aarch64-only,
    # simd.rs:220-228), and attention, norms and RoPE are per row: a pass of
    # m rows is its tokens one at a time, bit for bit, cache included.
    spec, layers, embed, final, cos_t, sin_t = _two_layer_model(False)
    one = O.Llm(spec, layers, embed, final, None, cos_t, sin_t)
    rows = O.Llm(spec, layers, embed, final, None, cos_t, sin_t)
    for t in TOKENS:
        want = one.forward(t)
    got = rows.forward_rows(TOKENS)
    np.testing.assert_array_equal(got, want)
    for l in range(spec["n_layer"]):
        np.testing.assert_array_equal(rows.kc[l], one.kc[l])
        np.testing.assert_array_equal(rows.vc[l], one.vc[l])
    # and a prompt in passes of three (batched_decode.rs:261-290's shape)
    passes = O.Llm(spec, layers, embed, final, None, cos_t, sin_t)
    np.testing.assert_array_equal(passes.forward_tokens(TOKENS, chunk=3), want)
    assert passes.len == rows.len == one.len == len(TOKENS)


@pytest.mark.parametrize("interleaved", [False, True])
def test_a_pass_is_the_float64_composition(interleaved):
    spec, layers, embed, final, cos_t, sin_t = _two_layer_model(interleaved)
    want = _f64_llm(spec, layers, embed, final, embed, cos_t, sin_t, TOKENS)[-1]
    got = O.Llm(spec, layers, embed, final, None, cos_t, sin_t).forward_rows(TOKENS)
    err = float(np.max(np.abs(got.astype(np.float64) - want))) / float(np.max(np.abs(want)))
    assert err <= 1e-5, err


def test_a_pass_catches_a_row_attending_past_itself():
    # a pass whose rows all attend over the whole pass (no causal mask) is
    # caught by the float64 composition: the bar above is not loose enough to
    # hide a wrong mask
    spec, layers, embed, final, cos_t, sin_t = _two_layer_model(False)
    want = _f64_llm(spec, layers, embed, final, embed, cos_t, sin_t, TOKENS)[-2]
    ref = O.Llm(spec, layers, embed, final, None, cos_t, sin_t)
    # the second-to-last token's logits with every row seeing the last row's key
    ref.forward_rows(TOKENS)
    ref.len = 0
    m = len(TOKENS) - 1
    # rerun the first m tokens over the full cache the previous pass left
    bad = O.Llm(spec, layers, embed, final, None, cos_t, sin_t)
    bad.kc, bad.vc = [k.copy() for k in ref.kc], [v.copy() for v in ref.vc]
    orig_attend = O.attend

    def leaky(nh, nkv, hd, q, kc, vc, n, L=None):
        return orig_attend(nh, nkv, hd, q, bad.kc[leaky.layer][:len(TOKENS)].ravel(),
                           bad.vc[leaky.layer][:len(TOKENS)].ravel(), len(TOKENS), L=L)

    try:
        calls = []

        def counting(nh, nkv, hd, q, kc, vc, n, L=None):
            leaky.layer = (len(calls) // m) % spec["n_layer"]
            calls.append(n)
            return leaky(nh, nkv, hd, q, kc, vc, n, L)

        O.attend = counting
        got = bad.forward_rows(TOKENS[:m])
    finally:
        O.attend = orig_attend
    err = float(np.max(np.abs(got.astype(np.float64) - want))) / float(np.max(np.abs(want)))
    assert err > 1e-2, err

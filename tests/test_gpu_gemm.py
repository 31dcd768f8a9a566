"""GPU parity of the batched-prefill GEMM (Weight::matmul_bt, quant.rs:751-907;
tensor::gemm_bt, tensor.rs:102-186) against the CPU oracle, through the C ABI.

Bar: f32 outputs within 1e-5 x max|ref|.  The integer block dots inside the
MFMA kernel are pinned bit-exactly by a known-answer case whose scales are
exactly 1.0, so every output is an exact integer sum.  At the Llama-3-8B
prefill shape the oracle is too slow for the whole product, so the GPU result
is checked on a sampled grid of rows x tokens: each output element depends
only on its weight row and activation row, so the oracle runs on those rows
alone.
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

import kvad_amd as K  # noqa: E402  (fails loudly without libkvad_hip.so)

from test_gpu_gemv import close, make, say  # noqa: E402


def oracle_matmul(prec, parts, rows, cols, xs, m, bias=None):
    if prec == "q8":
        return O.matmul_q8(*parts, rows, cols, xs, m, bias)
    if prec == "q4":
        return O.matmul_q4(*parts, rows, cols, xs, m, bias)
    if prec == "q4k":
        return O.matmul_q4k(parts[0], rows, cols, xs, m, bias)
    return O.matmul_f32(parts[0], rows, cols, xs, m, bias)


# (m tokens, rows, cols): edge tiles in every direction, k tails, tiny m
SHAPES = {
    "q8": [(2, 37, 64), (33, 130, 96), (65, 257, 288), (129, 128, 128), (3, 4864, 896)],
    "q4": [(2, 37, 64), (33, 130, 96), (65, 257, 288), (129, 128, 128)],
    "q4k": [(2, 37, 256), (33, 130, 512), (65, 257, 768), (129, 128, 256)],
    "f32": [(2, 3, 8), (33, 130, 100), (65, 257, 36), (7, 9, 13), (129, 128, 128)],
}


@pytest.mark.parametrize("prec", ["q8", "q4", "q4k", "f32"])
def test_matmul_matches_the_oracle(ctx, prec):
    for m, rows, cols in SHAPES[prec]:
        say("matmul", prec, m, rows, cols)
        w, parts = make(ctx, prec, rows, cols, seed=m + rows + cols)
        xs = O.normal(m * 3 + rows, m * cols)
        close(w.matmul_bt(xs, m), oracle_matmul(prec, parts, rows, cols, xs, m))
        bias = O.normal(rows + 5, rows)
        close(w.matmul_bt(xs, m, bias), oracle_matmul(prec, parts, rows, cols, xs, m, bias))


@pytest.mark.parametrize("tile", ["32", "64", "128", "6464"])
@pytest.mark.parametrize("prec", ["q8", "q4", "q4k"])
def test_every_tile_shape_matches_the_oracle(ctx, monkeypatch, prec, tile):
    # 128 weight rows by 32 / 64 / 128 tokens, or 64 by 64 (KVAD_GEMM_TILE_M):
    # edge tiles in both directions, k tails, the k-stages split or not
    monkeypatch.setenv("KVAD_GEMM_TILE_M", tile)
    for m, rows, cols in [(33, 130, 96 if prec != "q4k" else 256), (65, 257, 288 if prec != "q4k" else 768),
                          (40, 129, 192 if prec != "q4k" else 512), (100, 200, 1024)]:
        w, parts = make(ctx, prec, rows, cols, seed=m + 2 * rows + cols)
        xs = O.normal(m * 5 + rows, m * cols)
        bias = O.normal(rows + 9, rows)
        want = oracle_matmul(prec, parts, rows, cols, xs, m, bias)
        for ks in ("", "3"):
            say("matmul tile", prec, tile, m, rows, cols, ks or "auto")
            monkeypatch.setenv("KVAD_GEMM_KSPLIT", ks)
            close(w.matmul_bt(xs, m, bias), want)


@pytest.mark.parametrize("prec", ["q8", "f32"])
def test_qwen_prefill_shape(ctx, prec):
    # M = 512 tokens, K = 896, N = 4864
    m, rows, cols = 512, 4864, 896
    say("matmul qwen", prec)
    w, parts = make(ctx, prec, rows, cols, seed=42)
    xs = O.normal(7, m * cols)
    close(w.matmul_bt(xs, m), oracle_matmul(prec, parts, rows, cols, xs, m))


# (m tokens, rows, cols) with fewer tiles than CUs and at least four k-stages
# of 128: the k-stages split over the grid and the last split of each tile
# adds the others' partials; rows not a multiple of 4 take the scalar tail
SPLIT_SHAPES = [(32, 896, 4864), (100, 257, 1024), (9, 130, 2048), (128, 896, 4864)]


@pytest.mark.parametrize("prec", ["q8", "q4", "q4k"])
def test_split_k_matches_the_oracle(ctx, prec, monkeypatch):
    for m, rows, cols in SPLIT_SHAPES:
        w, parts = make(ctx, prec, rows, cols, seed=m + rows)
        xs = O.normal(m + 1, m * cols)
        bias = O.normal(rows + 2, rows)
        want = oracle_matmul(prec, parts, rows, cols, xs, m, bias)
        for ks in ("", "1", "3", "16"):  # automatic, none, forced
            say("matmul split-k", prec, m, rows, cols, ks or "auto")
            monkeypatch.setenv("KVAD_GEMM_KSPLIT", ks)
            got = w.matmul_bt(xs, m, bias)
            close(got, want)
            np.testing.assert_array_equal(w.matmul_bt(xs, m, bias), got)  # the same order every call


def test_split_k_partials_of_exact_integers_are_exact(ctx, monkeypatch):
    # scale-1 q8 blocks (the block maximum sits where the other operand is 0)
    # and small activation codes: every partial and every sum of partials is
    # an integer below 2^24, so however the k-stages split the result is the
    # exact integer product
    rng = np.random.default_rng(5)
    m, rows, cols = 70, 150, 4096
    x = rng.integers(-3, 4, size=(m, cols)).astype(np.float32)
    x[:, ::32] = 127.0
    wi = rng.integers(-127, 128, size=(rows, cols)).astype(np.float32)
    wi[:, ::32] = 0.0
    wi[:, 5::32] = -127.0
    s, q = O.quantize_q8(wi.ravel(), rows, cols)
    assert np.all(s == 1.0)
    w = K.Weight.from_q8(ctx, rows, cols, s, q)
    want = (x.astype(np.int64) @ q.reshape(rows, cols).astype(np.int64).T).astype(np.float64)
    assert np.max(np.abs(want)) < 2**24
    for ks in ("1", "2", "5", "16", "32"):
        say("split-k exact", ks)
        monkeypatch.setenv("KVAD_GEMM_KSPLIT", ks)
        got = w.matmul_bt(x.ravel(), m).reshape(m, rows)
        np.testing.assert_array_equal(got.astype(np.float64), want)


@pytest.mark.parametrize("prec", ["q8", "q4", "q4k"])
def test_integer_block_dots_are_exact(ctx, prec):
    # Weights and activations whose every block holds its extreme (+-127 for
    # q8 and the activations, -8 for q4), so each block scale is exactly 1.0
    # (q4: -8/-8) and y is the exact integer dot product -- any lane-layout or
    # block-boundary slip in the MFMA path changes it.
    rng = np.random.default_rng(3)
    m, rows, cols = 70, 150, 512
    say("exact dots", prec)
    x = rng.integers(-127, 128, size=(m, cols)).astype(np.float32)
    x[:, ::32] = 127.0
    if prec == "q8":
        wi = rng.integers(-127, 128, size=(rows, cols)).astype(np.float32)
        wi[:, 5::32] = -127.0
        s, q = O.quantize_q8(wi.ravel(), rows, cols)
        assert np.all(s == 1.0)
        w = K.Weight.from_q8(ctx, rows, cols, s, q)
        ref_w = q.reshape(rows, cols).astype(np.int64)
    elif prec == "q4":
        wi = rng.integers(-8, 8, size=(rows, cols)).astype(np.float32)
        wi[:, 3::32] = -8.0
        s, q = O.quantize_q4(wi.ravel() * 1.0, rows, cols)
        assert np.all(s == 1.0)
        w = K.Weight.from_q4(ctx, rows, cols, s, q)
        ref_w = wi.astype(np.int64)
    else:
        # Q4_K with d = 1, dmin = 0, every 6-bit scale 1: w = code, 0..15
        codes = rng.integers(0, 16, size=(rows, cols)).astype(np.uint8)
        blocks = np.zeros((rows, cols // 256, 144), np.uint8)
        blocks[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
        blocks[:, :, 4:8] = 1       # sc of sub-blocks 0..3
        blocks[:, :, 12:16] = 0x01  # sc of sub-blocks 4..7 (low nibble), m = 0
        cb = codes.reshape(rows, cols // 256, 4, 2, 32)  # [.., chunk c, nibble, l]
        blocks[:, :, 16:] = (cb[:, :, :, 0, :] | (cb[:, :, :, 1, :] << 4)).reshape(rows, cols // 256, 128)
        w = K.Weight.from_q4k(ctx, rows, cols, blocks.ravel())
        np.testing.assert_array_equal(w.row(1), codes[1].astype(np.float32))
        ref_w = codes.astype(np.int64)
    want = (x.astype(np.int64) @ ref_w.T).astype(np.float64)
    assert np.max(np.abs(want)) < 2**24
    got = w.matmul_bt(x.ravel(), m).reshape(m, rows)
    np.testing.assert_array_equal(got.astype(np.float64), want)


@pytest.mark.parametrize("prec", ["q8", "q4", "q4k", "f32"])
def test_batched_agrees_with_row_by_row(ctx, prec):
    # quant.rs:1305-1329: the batched product against one matvec per token
    m, rows, cols = 9, 96, 512
    say("batched vs rows", prec)
    w, parts = make(ctx, prec, rows, cols, seed=11)
    xs = O.normal(12, m * cols)
    got = w.matmul_bt(xs, m).reshape(m, rows)
    for i in range(m):
        close(got[i], w.matvec_bt(xs[i * cols:(i + 1) * cols]))
    one = w.matmul_bt(xs[:cols], 1)
    np.testing.assert_array_equal(one, w.matvec_bt(xs[:cols]))  # m == 1 is matvec, quant.rs:767-769


@pytest.mark.parametrize("prec", ["q8", "f32"])
def test_matmul_is_deterministic(ctx, prec):
    m, rows, cols = 300, 640, 1024
    say("matmul determinism", prec)
    w, _ = make(ctx, prec, rows, cols, seed=13)
    xs = O.normal(14, m * cols)
    first = w.matmul_bt(xs, m)
    for _ in range(3):
        np.testing.assert_array_equal(w.matmul_bt(xs, m), first)


@pytest.mark.parametrize("prec", ["q8", "q4k", "f32"])
def test_llama_prefill_shape_on_a_sampled_grid(ctx, prec):
    # M = 2048 tokens, K = 4096, N = 14336
    m, rows, cols = 2048, 14336, 4096
    say("matmul llama sampled", prec)
    wf = O.normal(21, rows * cols, 0.02)
    if prec == "q8":
        s, q = O.quantize_q8(wf, rows, cols)
        w = K.Weight.from_q8(ctx, rows, cols, s, q)
    elif prec == "q4k":
        b = O.quantize_q4k(wf, rows, cols)
        w = K.Weight.from_q4k(ctx, rows, cols, b)
    else:
        w = K.Weight.from_f32(ctx, wf.reshape(rows, cols))
    xs = O.normal(22, m * cols)
    got = w.matmul_bt(xs, m).reshape(m, rows)
    r_idx = np.r_[0:64, 7000:7064, rows - 64:rows]
    t_idx = np.r_[0:16, 1000:1016, m - 16:m]
    sub_x = xs.reshape(m, cols)[t_idx].ravel()
    nr = len(r_idx)
    if prec == "q8":
        sub = oracle_matmul("q8", (s.reshape(rows, -1)[r_idx].ravel(), q.reshape(rows, cols)[r_idx].ravel()),
                            nr, cols, sub_x, len(t_idx))
    elif prec == "q4k":
        sub = oracle_matmul("q4k", (b.reshape(rows, -1)[r_idx].ravel(),), nr, cols, sub_x, len(t_idx))
    else:
        sub = oracle_matmul("f32", (wf.reshape(rows, cols)[r_idx].ravel(),), nr, cols, sub_x, len(t_idx))
    close(got[np.ix_(t_idx, r_idx)], sub.reshape(len(t_idx), nr))
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("m", [2, 16])
def test_two_by_two_known_answer(ctx, m):
    # The reference's SMMLA known answer (simd.rs:236-261): A0 = 1..8,
    # A1 = ones, B0 = ones, B1 = 0,...,0,10 gives [A0.B0, A0.B1, A1.B0, A1.B1]
    # = [36, 80, 8, 10].  Here through matmul_bt: weight codes as given with
    # scale 1, activations whose block maximum is 127 (column 31, where the
    # weights are 0) so their codes are the values themselves and their scale
    # is 1.  m = 2 runs the multi-token GEMV, m = 16 the MFMA GEMM (rows
    # repeated); the products sit in y[token][row].
    say("matmul 2x2 known answer", m)
    a = np.zeros((2, 32), np.int8)
    a[0, :8] = np.arange(1, 9)
    a[1, :8] = 1
    w = K.Weight.from_q8(ctx, 2, 32, np.ones(2, np.float32), a.ravel())
    x = np.zeros((2, 32), np.float32)
    x[0, :8] = 1.0
    x[1, 7] = 10.0
    x[:, 31] = 127.0
    xs = np.tile(x, (m // 2, 1))
    y = w.matmul_bt(xs.ravel(), m).reshape(m, 2)
    want = np.tile(np.array([[36.0, 8.0], [80.0, 10.0]], np.float32), (m // 2, 1))
    np.testing.assert_array_equal(y, want)


@pytest.mark.parametrize("prec", ["q8", "q4k"])
@pytest.mark.parametrize("m", [3, 8])
def test_few_tokens_over_a_wide_activation(ctx, prec, m):
    # the multi-token GEMV with Llama-3-8B's 14336-wide down-projection input:
    # eight token slots of it need a stage past 64 KB of LDS (up to 160 KB)
    rows, cols = 64, 14336
    say("matmul wide", prec, m)
    w, parts = make(ctx, prec, rows, cols, seed=rows + m)
    xs = O.normal(m + 99, m * cols)
    close(w.matmul_bt(xs, m), oracle_matmul(prec, parts, rows, cols, xs, m))

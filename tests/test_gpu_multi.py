"""GPU parity of matmul_bt at a few tokens (batched decode: Weight::matmul_bt,
quant.rs:751-907, as forward_each calls it, llama.rs:418-434), which the
library runs as a multi-token GEMV that streams the weights once for every
token: on the VALU (dot4 per row and token; two token rows, or any with
KVAD_MMA_MIN above m) or on the matrix cores (one v_mfma_i32_16x16x32_i8
per block pair for 16 rows x 8 tokens, per block for 16 tokens; from five
token rows).

Bar: f32 outputs within 1e-5 x max|ref| of the oracle's matmul.  On the VALU
path each token's row equals, to the bit, a single-token matvec of that
token (the per-token arithmetic is the GEMV's, term for term); on the matrix
cores the exact i32 block dots are scaled and summed in another order, so
the row is held to 1e-5 x max|row| of the matvec.  Shapes cover ragged row
counts (a last 16-row group part-filled), k tails (widths not a multiple of
four blocks), rows of one and of several segments, widths whose staged
codes take more than one launch of token slots, and, on the matrix cores,
more than 16 tokens (a launch per 16).
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

import kvad_amd as K  # noqa: E402  (fails loudly without libkvad_hip.so)

from test_gpu_gemm import oracle_matmul  # noqa: E402
from test_gpu_gemv import close, make, say  # noqa: E402

# (rows, cols) per precision: ragged rows, one segment, several segments,
# Qwen2.5-0.5B FFN shapes, a Llama-3-8B down row width
SHAPES = {
    "q8": [(37, 64), (130, 2048), (4864, 896), (896, 4864)],
    "q4": [(37, 64), (130, 2048), (896, 4864)],
    "q4k": [(37, 256), (130, 4096), (300, 14336)],
}


PATHS = {"valu": "99", "mma": "2"}  # KVAD_MMA_MIN: the matrix cores from this many rows


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("prec", ["q8", "q4", "q4k"])
@pytest.mark.parametrize("m", [2, 3, 4, 5, 8])
def test_few_tokens_match_the_oracle_and_single_matvecs(ctx, monkeypatch, path, prec, m):
    monkeypatch.setenv("KVAD_MMA_MIN", PATHS[path])
    for rows, cols in SHAPES[prec]:
        say("multi-token matmul", path, prec, m, rows, cols)
        w, parts = make(ctx, prec, rows, cols, seed=rows + cols + m)
        xs = O.normal(rows * 7 + m, m * cols)
        bias = O.normal(rows + 3, rows)
        for b in (None, bias):
            got = w.matmul_bt(xs, m, b)
            close(got, oracle_matmul(prec, parts, rows, cols, xs, m, b))
            got = got.reshape(m, rows)
            for t in range(m):
                one = w.matvec_bt(xs[t * cols:(t + 1) * cols], b)
                if path == "valu":
                    np.testing.assert_array_equal(got[t], one)
                else:
                    close(got[t], one)


# the matrix cores: ragged 16-row groups, k tails of 1..3 blocks past whole
# four-block units, Q4_K's minimum terms over several super-blocks, and
# Qwen2.5-0.5B / Llama-3-8B widths
MMA_SHAPES = {
    "q8": [(1, 32), (17, 96), (37, 160), (130, 2048), (896, 4864), (64, 14336)],
    "q4": [(1, 32), (17, 96), (37, 224), (130, 2048), (896, 4864)],
    "q4k": [(1, 256), (17, 768), (130, 4096), (64, 14336)],
}


@pytest.mark.parametrize("prec", ["q8", "q4", "q4k"])
@pytest.mark.parametrize("m", [3, 8, 9, 16, 17, 40])
def test_matrix_core_tokens_match_the_oracle(ctx, monkeypatch, prec, m):
    # up to 40 rows through the matrix-core path (KVAD_MULTI_TOKENS,
    # KVAD_MMA_MIN): block pairs up to 8 rows, a block per instruction from 9;
    # 17 and 40 take a launch per 16 rows, each writing its own rows of y
    monkeypatch.setenv("KVAD_MULTI_TOKENS", "64")
    monkeypatch.setenv("KVAD_MMA_MIN", "2")
    for rows, cols in MMA_SHAPES[prec]:
        say("matrix-core matmul", prec, m, rows, cols)
        w, parts = make(ctx, prec, rows, cols, seed=3 * rows + cols + m)
        xs = O.normal(rows * 5 + m, m * cols)
        bias = O.normal(rows + 7, rows)
        for b in (None, bias):
            close(w.matmul_bt(xs, m, b), oracle_matmul(prec, parts, rows, cols, xs, m, b))


def test_many_token_slots_stream_in_launches(ctx, monkeypatch):
    # the VALU path, 8 tokens at a width whose codes fill the LDS stage for 2
    # at a time
    monkeypatch.setenv("KVAD_MMA_MIN", "99")
    rows, cols, m = 64, 14336, 8
    say("multi-token matmul, staged in launches")
    w, parts = make(ctx, "q4k", rows, cols, seed=5)
    xs = O.normal(6, m * cols)
    got = w.matmul_bt(xs, m)
    close(got, oracle_matmul("q4k", parts, rows, cols, xs, m))


@pytest.mark.parametrize("path", list(PATHS))
def test_zero_and_edge_tokens(ctx, monkeypatch, path):
    # a token of zeros quantises to zero codes (scale 0): its row is the bias
    monkeypatch.setenv("KVAD_MMA_MIN", PATHS[path])
    rows, cols, m = 96, 512, 3
    w, parts = make(ctx, "q8", rows, cols, seed=9)
    xs = O.normal(10, m * cols)
    xs[cols:2 * cols] = 0.0
    bias = O.normal(11, rows)
    got = w.matmul_bt(xs, m, bias).reshape(m, rows)
    np.testing.assert_array_equal(got[1], bias.astype(np.float32))
    close(got.ravel(), oracle_matmul("q8", parts, rows, cols, xs, m, bias))

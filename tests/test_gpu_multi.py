"""GPU parity of matmul_bt at a few tokens (batched decode: Weight::matmul_bt,
quant.rs:751-907, as forward_each calls it, llama.rs:418-434), which the
library runs as a multi-token GEMV that streams the weights once for every
token.

Bar: f32 outputs within 1e-5 x max|ref| of the oracle's matmul, and each
token's row equal, to the bit, to a single-token matvec of that token (the
per-token arithmetic is the GEMV's, term for term).  Shapes cover ragged row
counts, rows of one and of several segments, and widths whose staged codes
take more than one launch of token slots.
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


@pytest.mark.parametrize("prec", ["q8", "q4", "q4k"])
@pytest.mark.parametrize("m", [2, 3, 4, 5, 8])
def test_few_tokens_match_the_oracle_and_single_matvecs(ctx, prec, m):
    for rows, cols in SHAPES[prec]:
        say("multi-token matmul", prec, m, rows, cols)
        w, parts = make(ctx, prec, rows, cols, seed=rows + cols + m)
        xs = O.normal(rows * 7 + m, m * cols)
        bias = O.normal(rows + 3, rows)
        for b in (None, bias):
            got = w.matmul_bt(xs, m, b)
            close(got, oracle_matmul(prec, parts, rows, cols, xs, m, b))
            got = got.reshape(m, rows)
            for t in range(m):
                np.testing.assert_array_equal(got[t], w.matvec_bt(xs[t * cols:(t + 1) * cols], b))


def test_many_token_slots_stream_in_launches(ctx):
    # 8 tokens at a width whose codes fill the LDS stage for 2 at a time
    rows, cols, m = 64, 14336, 8
    say("multi-token matmul, staged in launches")
    w, parts = make(ctx, "q4k", rows, cols, seed=5)
    xs = O.normal(6, m * cols)
    got = w.matmul_bt(xs, m)
    close(got, oracle_matmul("q4k", parts, rows, cols, xs, m))


def test_zero_and_edge_tokens(ctx):
    # a token of zeros quantises to zero codes (scale 0): its row is the bias
    rows, cols, m = 96, 512, 3
    w, parts = make(ctx, "q8", rows, cols, seed=9)
    xs = O.normal(10, m * cols)
    xs[cols:2 * cols] = 0.0
    bias = O.normal(11, rows)
    got = w.matmul_bt(xs, m, bias).reshape(m, rows)
    np.testing.assert_array_equal(got[1], bias.astype(np.float32))
    close(got.ravel(), oracle_matmul("q8", parts, rows, cols, xs, m, bias))

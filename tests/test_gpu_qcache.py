"""Cache-file weights uploaded to the device (kh_qcache_weight, Mapped::build
qcache.rs:689-713): the device arrays equal the file's bytes, and the mapped
weight gives bit-identical answers to the same weight built from arrays --
the reference's round-trip criterion (qcache.rs:1499-1532: "bit-identical
answers, not close ones").  GGML Q8_0/Q4_0 blocks repack to kvad's layout
exactly (f16 -> f32 scales), checked against the oracle's q8/q4 matvec."""
import numpy as np
import pytest

import kvad_amd as K
import oracle as O
from nanoq import Writer, ggml_q4_0, ggml_q8_0

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cache(tmp_path_factory):
    path = tmp_path_factory.mktemp("qc") / "w.nanoq"
    w = Writer(path)
    arrays = {}
    rows, cols = 96, 512
    data = O.normal(11, rows * cols, 0.02)
    s8, q8 = O.quantize_q8(data, rows, cols)
    s4, q4 = O.quantize_q4(data, rows, cols)
    w.q8("q8", rows, cols, s8, q8)
    w.q4("q4", rows, cols, s4, q4)
    w.f32("f32", data, rows, cols)
    blocks = O.quantize_q4k(data, rows, cols)
    w.ggml("q4k", "q4k", rows, cols, blocks)
    f16 = np.array([O.f32_to_f16(float(v)) for v in s8], np.uint16)
    w.ggml("g8", "q8", rows, cols, ggml_q8_0(f16, q8))
    w.ggml("g4", "q4", rows, cols, ggml_q4_0(f16, q4))
    # large enough for several 16 MiB staging chunks, with GGML blocks
    # straddling chunk boundaries
    br, bc = 2048, 12288
    big = O.normal(12, br * bc, 0.02)
    bs8, bq8 = O.quantize_q8(big, br, bc)
    bf16 = np.array([O.f32_to_f16(float(v)) for v in bs8[:4096]] * (bs8.size // 4096), np.uint16)
    w.q8("big", br, bc, bs8, bq8)
    w.ggml("gbig", "q8", br, bc, ggml_q8_0(bf16, bq8))
    w.finish()
    arrays.update(rows=rows, cols=cols, data=data, s8=s8, q8=q8, s4=s4, q4=q4, blocks=blocks, f16=f16,
                  br=br, bc=bc, bs8=bs8, bq8=bq8, bf16=bf16)
    return K.QCache(path), arrays


def test_device_arrays_equal_the_file(ctx, cache):
    qc, a = cache
    sc, qs = qc.weight(ctx, "q8").parts()
    assert np.array_equal(sc.view(np.uint32), a["s8"].view(np.uint32)) and np.array_equal(qs, a["q8"])
    sc, qs = qc.weight(ctx, "q4").parts()
    assert np.array_equal(sc.view(np.uint32), a["s4"].view(np.uint32)) and np.array_equal(qs, a["q4"])
    _, qs = qc.weight(ctx, "q4k").parts()
    assert np.array_equal(qs, a["blocks"])
    _, qs = qc.weight(ctx, "f32").parts()
    assert np.array_equal(qs.view(np.uint32), a["data"].view(np.uint32))
    sc, qs = qc.weight(ctx, "big").parts()
    assert np.array_equal(sc.view(np.uint32), a["bs8"].view(np.uint32)) and np.array_equal(qs, a["bq8"])


def test_mapped_weights_answer_bit_identically(ctx, cache):
    qc, a = cache
    rows, cols = a["rows"], a["cols"]
    x = np.sin(np.arange(cols, dtype=np.float32))
    built = {
        "q8": K.Weight.from_q8(ctx, rows, cols, a["s8"], a["q8"]),
        "q4": K.Weight.from_q4(ctx, rows, cols, a["s4"], a["q4"]),
        "q4k": K.Weight.from_q4k(ctx, rows, cols, a["blocks"]),
        "f32": K.Weight.from_f32(ctx, a["data"].reshape(rows, cols)),
    }
    for name, w in built.items():
        m = qc.weight(ctx, name)
        assert np.array_equal(m.matvec_bt(x), w.matvec_bt(x)), name
        assert np.array_equal(m.row(3), w.row(3)), name  # the embedding path


def test_ggml_blocks_repack_exactly(ctx, cache):
    qc, a = cache
    rows, cols = a["rows"], a["cols"]
    scales = np.array([O.f16_to_f32(int(h)) for h in a["f16"]], np.float32)
    sc, qs = qc.weight(ctx, "g8").parts()
    assert np.array_equal(sc, scales) and np.array_equal(qs, a["q8"])
    sc, qs = qc.weight(ctx, "g4").parts()
    assert np.array_equal(sc, scales) and np.array_equal(qs, a["q4"])
    x = O.normal(13, cols)
    y8 = qc.weight(ctx, "g8").matvec_bt(x)
    want8 = O.matvec_q8(scales, a["q8"], rows, cols, x)
    assert np.max(np.abs(y8 - want8)) <= 1e-5 * np.max(np.abs(want8))
    y4 = qc.weight(ctx, "g4").matvec_bt(x)
    want4 = O.matvec_q4(scales, a["q4"], rows, cols, x)
    assert np.max(np.abs(y4 - want4)) <= 1e-5 * np.max(np.abs(want4))
    # several staging chunks, block boundaries across them
    sc, qs = qc.weight(ctx, "gbig").parts()
    bsc = np.array([O.f16_to_f32(int(h)) for h in a["bf16"][:4096]], np.float32)
    assert np.array_equal(sc, np.tile(bsc, sc.size // 4096)) and np.array_equal(qs, a["bq8"])


def test_a_missing_name_is_an_error(ctx, cache):
    qc, _ = cache
    with pytest.raises(K.KvadError, match="no tensor"):
        qc.weight(ctx, "nope")

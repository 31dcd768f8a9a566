"""The quantised-weight cache container (crates/llm/src/qcache.rs) as the
library parses it: no device needed.  Cases follow the reference's own tests
(qcache.rs:1499-1617): weights and vectors survive the round trip, a file that
is not one of ours is refused, and spans are checked against the file
(Container::slice, qcache.rs:906-911)."""
import json
import struct

import numpy as np
import pytest

import kvad_amd as K
import oracle as O
from nanoq import Writer, ggml_q4_0, ggml_q8_0


def _write_all(path):
    w = Writer(path)
    rows, cols = 8, 64
    data = np.array([((i * 37 % 101) - 50.0) / 25.0 for i in range(rows * cols)], np.float32)
    s8, q8 = O.quantize_q8(data, rows, cols)
    s4, q4 = O.quantize_q4(data, rows, cols)
    w.q8("a8", rows, cols, s8, q8)
    w.q4("a4", rows, cols, s4, q4)
    w.f32("norm", [1.0, 2.0, 3.0])
    w.f32("dense", data, rows, cols)
    blocks = O.quantize_q4k(O.normal(5, 4 * 256, 0.02), 4, 256)
    w.ggml("k4", "q4k", 4, 256, blocks)
    f16 = np.array([O.f32_to_f16(0.01 * (i + 1)) for i in range(rows * cols // 32)], np.uint16)
    w.ggml("g8", "q8", rows, cols, ggml_q8_0(f16, q8))
    w.ggml("g4", "q4", rows, cols, ggml_q4_0(f16, q4))
    w.ggml("g6", "q6k", 4, 256, np.zeros(4 * 210, np.uint8))  # no device kernel: left out
    w.finish({"version": 2, "precision": "q8", "repo": "r", "checkpoint": ["a8", "a4"]})
    return dict(rows=rows, cols=cols, data=data, s8=s8, q8=q8, s4=s4, q4=q4, blocks=blocks, f16=f16)


def test_entries_survive_the_round_trip(tmp_path):
    path = tmp_path / "rt.nanoq"
    _write_all(path)
    qc = K.QCache(path)
    assert qc.names() == ["a8", "a4", "norm", "dense", "k4", "g8", "g4"]
    assert qc.info("a8") == (K.Q8, 8, 64)
    assert qc.info("a4") == (K.Q4, 8, 64)
    assert qc.info("dense") == (K.F32, 8, 64)
    assert qc.info("k4") == (K.Q4K, 4, 256)
    assert qc.info("g8") == (K.Q8, 8, 64)  # GGML Q8_0, repacked on upload
    assert qc.info("g4") == (K.Q4, 8, 64)
    assert qc.vector("norm").tolist() == [1.0, 2.0, 3.0]
    h = json.loads(qc.header())
    assert h["repo"] == "r" and h["checkpoint"] == ["a8", "a4"] and set(h["tensors"]) >= {"a8", "g6"}
    with pytest.raises(K.KvadError):
        qc.info("g6")
    with pytest.raises(K.KvadError):
        qc.vector("dense")  # a matrix, not a vector (Mapped::vector wants shape [1, n])
    qc.close()


def test_header_strings_and_numbers_of_every_form(tmp_path):
    path = tmp_path / "json.nanoq"
    w = Writer(path)
    w.f32("vé\"x\\", [0.5])
    w.finish({"version": 2, "note": "tab\tnew\nline ☃ \U0001F600", "pi": 3.25e0, "neg": -7, "ok": True,
              "none": None, "nested": {"a": [1, [2, {"b": []}]], "c": {}}})
    qc = K.QCache(path)
    assert qc.names() == ["vé\"x\\"]
    assert qc.vector("vé\"x\\").tolist() == [0.5]
    assert json.loads(qc.header())["note"] == "tab\tnew\nline ☃ \U0001F600"


def test_a_file_that_is_not_one_of_ours_is_refused(tmp_path):
    junk = tmp_path / "junk"
    junk.write_bytes(bytes([7]) * 256)  # qcache.rs:1583-1586
    with pytest.raises(K.KvadError, match="not a quantised-weight file"):
        K.QCache(junk)
    short = tmp_path / "short"
    short.write_bytes(b"NANOQ\x00\x00\x01")
    with pytest.raises(K.KvadError):
        K.QCache(short)
    with pytest.raises(K.KvadError, match="cannot open"):
        K.QCache(tmp_path / "absent")


def _good(tmp_path):
    path = tmp_path / "good.nanoq"
    w = Writer(path)
    w.f32("x", np.arange(16, dtype=np.float32))
    w.finish()
    return path, bytearray(path.read_bytes())


def test_the_trailer_and_header_are_checked(tmp_path):
    path, b = _good(tmp_path)
    bad = tmp_path / "bad"
    # header offset pointing past the end, or into the first 64 bytes
    for at in (len(b), 8):
        c = bytearray(b)
        c[-8:] = struct.pack("<Q", at)
        bad.write_bytes(c)
        with pytest.raises(K.KvadError, match="header offset"):
            K.QCache(bad)
    # a header that is not JSON
    at = struct.unpack("<Q", bytes(b[-8:]))[0]
    c = bytearray(b)
    c[at] = ord("[") if c[at] != ord("[") else ord("{")
    c[at + 1:at + 2] = b"!"
    bad.write_bytes(c)
    with pytest.raises(K.KvadError, match="not JSON"):
        K.QCache(bad)


def test_spans_past_the_end_of_the_file_are_refused(tmp_path):
    path = tmp_path / "trunc.nanoq"
    w = Writer(path)
    off = w.put(np.zeros(4, np.float32))
    w.tensors["x"] = {"kind": "f32", "shape": [1, 4], "data": [off[0], 1 << 40]}
    w.finish()
    with pytest.raises(K.KvadError, match="span length|past the end"):
        K.QCache(path)
    w = Writer(path)
    w.put(np.zeros(4, np.float32))
    w.tensors["x"] = {"kind": "q8", "shape": [1, 32], "scales": [len(w.buf) + 10_000, 1], "qs": [64, 32]}
    w.finish()
    with pytest.raises(K.KvadError, match="past the end"):
        K.QCache(path)


@pytest.mark.parametrize("entry, why", [
    ({"kind": "q8", "shape": [2, 33], "scales": [64, 2], "qs": [64, 66]}, "multiple of 32"),
    ({"kind": "q8", "shape": [2, 32], "scales": [64, 3], "qs": [64, 64]}, "does not match"),
    ({"kind": "f32", "shape": [2], "data": [64, 2]}, "shape"),
    ({"shape": [1, 1], "data": [64, 1]}, "kind"),
    ({"kind": "f32", "shape": [1, 1], "data": [64]}, "span"),
    ({"kind": "q4k", "shape": [1, 300], "data": [64, 144]}, "multiple of the block"),
])
def test_malformed_entries_are_refused(tmp_path, entry, why):
    path = tmp_path / "bad.nanoq"
    w = Writer(path)
    w.put(np.zeros(64, np.float32))
    w.tensors["t"] = entry
    w.finish()
    with pytest.raises(K.KvadError, match=why):
        K.QCache(path)

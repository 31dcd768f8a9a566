"""Writes quantised-weight cache files ("NANOQ") for the tests: a restatement
of the reference's Writer (crates/llm/src/qcache.rs:932-1040) -- magic, 56
reserved bytes, every array padded to a 64-byte boundary and described by a
[byte offset, element count] span, the JSON header after the last array, and
the header's offset as a little-endian u64 at the very end.  Entries are the
CPU engine's (put_weight / put_vector, qcache.rs:986-1018) or the GPU
backend's GGML blocks (crates/gpu/src/qcache.rs:278-296)."""
from __future__ import annotations

import json
import struct

import numpy as np

MAGIC = b"NANOQ\x00\x00\x01"
ALIGN = 64


class Writer:
    def __init__(self, path):
        self.path = path
        self.buf = bytearray(MAGIC + bytes(ALIGN - 8))
        self.tensors: dict[str, dict] = {}

    def put(self, a: np.ndarray) -> list[int]:
        """Append one array at the next 64-byte boundary; its span."""
        self.buf += bytes((ALIGN - len(self.buf) % ALIGN) % ALIGN)
        off = len(self.buf)
        self.buf += np.ascontiguousarray(a).tobytes()
        return [off, int(a.size)]

    def q8(self, name, rows, cols, scales, qs):
        self.tensors[name] = {"kind": "q8", "shape": [rows, cols], "scales": self.put(np.asarray(scales, np.float32)),
                              "qs": self.put(np.asarray(qs, np.int8))}

    def q4(self, name, rows, cols, scales, qs):
        self.tensors[name] = {"kind": "q4", "shape": [rows, cols], "scales": self.put(np.asarray(scales, np.float32)),
                              "qs": self.put(np.asarray(qs, np.uint8))}

    def f32(self, name, a, rows=None, cols=None):
        a = np.asarray(a, np.float32)
        shape = [1, a.size] if rows is None else [rows, cols]
        self.tensors[name] = {"kind": "f32", "shape": shape, "data": self.put(a.ravel())}

    def ggml(self, name, kind, rows, cols, blocks):
        self.tensors[name] = {"kind": kind, "shape": [rows, cols], "data": self.put(np.asarray(blocks, np.uint8))}

    def finish(self, header: dict | None = None) -> None:
        h = dict(header or {"version": 2, "precision": "q8", "repo": "test/model"})
        h["tensors"] = self.tensors
        at = len(self.buf)
        self.buf += json.dumps(h).encode() + struct.pack("<Q", at)
        with open(self.path, "wb") as f:
            f.write(self.buf)


def ggml_q8_0(scales_f16: np.ndarray, codes: np.ndarray) -> np.ndarray:
    """block_q8_0: f16 d, then 32 int8 codes (GGML's layout)."""
    nb = scales_f16.size
    out = np.zeros((nb, 34), np.uint8)
    out[:, :2] = scales_f16.astype(np.uint16).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = codes.astype(np.int8).view(np.uint8).reshape(nb, 32)
    return out.ravel()


def ggml_q4_0(scales_f16: np.ndarray, nibbles: np.ndarray) -> np.ndarray:
    """block_q4_0: f16 d, then 16 bytes (byte j: element j low nibble, j+16 high)."""
    nb = scales_f16.size
    out = np.zeros((nb, 18), np.uint8)
    out[:, :2] = scales_f16.astype(np.uint16).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = nibbles.astype(np.uint8).reshape(nb, 16)
    return out.ravel()

"""kvad_amd -- MI355X (gfx950) implementation of kvad's quantised matmul and
decode attention, behind the C ABI in include/kvad_hip.h.

This module is a thin ctypes mirror of that ABI, shaped like the reference's
Rust operator API so that tests and benchmarks read like the reference's own:

    Weight.matvec_bt(x, bias)        quant.rs:481    Weight::matvec_bt
    Weight.matmul_bt(xs, m, bias)    quant.rs:751    Weight::matmul_bt
    Weight.row(r)                    quant.rs:374    Weight::row
    matvec_many(ctx, jobs)           quant.rs:628    quant::matvec_many
    KvCache.push/keys/truncate/...   model/mod.rs:612-749
    attend(ctx, spec, q, cache, layer, n)   model/mod.rs:769

There is no CPU fallback: if libkvad_hip.so is missing this import fails.
"""
from __future__ import annotations

import ctypes as C
import os
import weakref
from dataclasses import dataclass
from pathlib import Path

import numpy as np

__all__ = [
    "F32", "Q8", "Q4", "Q4K", "KvadError", "Declined", "lib", "Context", "Weight", "matvec_many",
    "KvCache", "Spec", "attend", "LIB_PATH", "Moe", "QCache", "mla_attend", "mla_attend_dev", "Llm", "LlmSpec", "Parked", "SOFTMAX", "SIGMOID", "GREEDY", "GROUP_LIMITED", "NOAUX_TC",
]

F32, Q8, Q4, Q4K = 0, 1, 2, 3
SOFTMAX, SIGMOID = 0, 1                   # Scoring, model/ffn.rs:173-177
GREEDY, GROUP_LIMITED, NOAUX_TC = 0, 1, 2  # Select, model/ffn.rs:179-195
OK, DECLINED = 0, 1

LIB_PATH = Path(os.environ.get("KVAD_HIP_LIB", Path(__file__).resolve().parent / "libkvad_hip.so"))


class KvadError(RuntimeError):
    """A negative status from the library, with kh_last_error()'s message."""


class Declined(KvadError):
    """Status 1: the library declines; the reference would run its CPU kernel."""


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python kvad_amd/build.py` "
            "(there is no CPU fallback for this path)")
    # torch ships its own HIP runtime under the same soname.  Loaded first, it
    # serves this library too, so a process that also uses torch for device
    # memory has one runtime; loaded second, it would start a second runtime
    # beside the system one and find no device.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    return C.CDLL(str(LIB_PATH))


lib = _load()

_p = C.c_void_p
_sz = C.c_size_t
_fp = C.POINTER(C.c_float)
_SIGS = {
    "kh_last_error": (C.c_char_p, []),
    "kh_version": (C.c_char_p, []),
    "kh_init": (C.c_int, [C.c_int, C.POINTER(_p)]),
    "kh_free": (C.c_int, [_p]),
    "kh_set_stream": (C.c_int, [_p, _p]),
    "kh_synchronize": (C.c_int, [_p]),
    "kh_reserve": (C.c_int, [_p, _sz]),
    "kh_weight_q8": (C.c_int, [_p, _sz, _sz, _p, _p, C.POINTER(_p)]),
    "kh_weight_q4": (C.c_int, [_p, _sz, _sz, _p, _p, C.POINTER(_p)]),
    "kh_weight_q4k": (C.c_int, [_p, _sz, _sz, _p, C.POINTER(_p)]),
    "kh_weight_f32": (C.c_int, [_p, _sz, _sz, _p, C.POINTER(_p)]),
    "kh_weight_quantize": (C.c_int, [_p, _sz, _sz, _p, C.c_int, C.POINTER(_p)]),
    "kh_weight_quantize_dev": (C.c_int, [_p, _sz, _sz, _p, C.c_int, C.POINTER(_p)]),
    "kh_weight_parts": (C.c_int, [_p, _p, _p]),
    "kh_weight_free": (C.c_int, [_p]),
    "kh_weight_info": (C.c_int, [_p, C.POINTER(_sz), C.POINTER(_sz), C.POINTER(C.c_int), C.POINTER(_sz)]),
    "kh_weight_row": (C.c_int, [_p, _p, _sz, _p]),
    "kh_matvec": (C.c_int, [_p, _p, _p, _p, _p]),
    "kh_matvec_dev": (C.c_int, [_p, _p, _p, _p, _p]),
    "kh_matvec_dequant": (C.c_int, [_p, _p, _p, _p, _p]),
    "kh_matvec_dequant_dev": (C.c_int, [_p, _p, _p, _p, _p]),
    "kh_matvec_many": (C.c_int, [_p, _sz, _p, _p, _p]),
    "kh_matvec_many_dev": (C.c_int, [_p, _sz, _p, _p, _p]),
    "kh_matmul": (C.c_int, [_p, _p, _p, _sz, _p, _p]),
    "kh_matmul_dev": (C.c_int, [_p, _p, _p, _sz, _p, _p]),
    "kh_qact_dev": (C.c_int, [_p, _p, _sz, _sz, _p, _p, _p]),
    "kh_matvec_q_dev": (C.c_int, [_p, _p, _p, _p, _p, _p, _p]),
    "kh_debug_block_dots": (C.c_int, [_p, _p, _p, _p]),
    "kh_debug_qact": (C.c_int, [_p, _p, _sz, _p, _p, _p]),
    "kh_debug_quant_check": (C.c_int, [_p, _p]),
    "kh_kv_new": (C.c_int, [_p, _sz, _sz, _sz, _sz, C.POINTER(_p)]),
    "kh_kv_free": (C.c_int, [_p]),
    "kh_kv_push": (C.c_int, [_p, _sz, _p, _p, _sz]),
    "kh_kv_push_dev": (C.c_int, [_p, _sz, _p, _p, _sz]),
    "kh_kv_len": (C.c_int, [_p, C.POINTER(_sz)]),
    "kh_kv_set_len": (C.c_int, [_p, _sz]),
    "kh_kv_truncate": (C.c_int, [_p, _sz, C.POINTER(_sz)]),
    "kh_kv_clear": (C.c_int, [_p]),
    "kh_kv_keys": (C.c_int, [_p, _sz, _p, C.POINTER(_sz)]),
    "kh_kv_values": (C.c_int, [_p, _sz, _p, C.POINTER(_sz)]),
    "kh_kv_layer_ptrs": (C.c_int, [_p, _sz, C.POINTER(_p), C.POINTER(_p)]),
    "kh_attend": (C.c_int, [_p, _p, _sz, _sz, _sz, _sz, _p, _sz, _p]),
    "kh_attend_dev": (C.c_int, [_p, _sz, _sz, _sz, _p, _p, _p, _sz, _p]),
    "kh_attend_dev_noalloc": (C.c_int, [_p, _sz, _sz, _sz, _p, _p, _p, _sz, _p]),
    "kh_noalloc_scratch_bytes": (_sz, []),
    "kh_rms_norm_dev": (C.c_int, [_p, _p, _p, _sz, _sz, C.c_float, _p]),
    "kh_rope_dev": (C.c_int, [_p, _p, _p, _sz, _p, _sz, _sz, _sz, C.c_int]),
    "kh_swiglu_dev": (C.c_int, [_p, _p, _p, _sz]),
    "kh_softmax_dev": (C.c_int, [_p, _p, _sz, _sz]),
    "kh_llm_new": (C.c_int, [_p, _p, C.POINTER(_p)]),
    "kh_llm_free": (C.c_int, [_p]),
    "kh_llm_set_layer": (C.c_int, [_p, _sz] + [_p] * 14),
    "kh_llm_set_ends": (C.c_int, [_p, _p, _p, _p]),
    "kh_llm_set_rope": (C.c_int, [_p, _p, _p, _sz]),
    "kh_llm_forward": (C.c_int, [_p, _p, C.c_int32, _p, _p]),
    "kh_debug_llm_trace": (C.c_int, [_p, _p, C.c_int32, _p]),
    "kh_llm_forward_tokens": (C.c_int, [_p, _p, _p, _sz, _p, _p]),
    "kh_debug_stream_dev": (C.c_int, [_p, _sz, _p, _p]),
    "kh_llm_prefill_pass": (C.c_int, [_p, _sz, C.POINTER(_sz)]),
    "kh_llm_set_prefill_chunk": (C.c_int, [_p, _sz]),
    "kh_debug_llm_trace_pass": (C.c_int, [_p, _p, _p, _sz, _p]),
    "kh_llm_generate": (C.c_int, [_p, _p, C.c_int32, _sz, _p]),
    "kh_llm_generate_launch": (C.c_int, [_p, _p, _sz]),
    "kh_llm_len": (C.c_int, [_p, C.POINTER(_sz)]),
    "kh_llm_truncate": (C.c_int, [_p, _sz]),
    "kh_llm_park": (C.c_int, [_p, C.POINTER(_p)]),
    "kh_llm_resume": (C.c_int, [_p, _p]),
    "kh_llm_parked_free": (C.c_int, [_p]),
    "kh_llm_parked_len": (C.c_int, [_p, C.POINTER(_sz)]),
    "kh_llm_forward_each": (C.c_int, [_p, _p, _sz, _p, _p, _p, _p]),
    "kh_moe_new": (C.c_int, [_p, _sz, _sz, _sz, _sz, C.c_int, C.c_int, _sz, _sz, C.c_int, C.c_float, _p,
                             C.POINTER(_p)]),
    "kh_moe_free": (C.c_int, [_p]),
    "kh_moe_set_router": (C.c_int, [_p, _p]),
    "kh_moe_set_expert": (C.c_int, [_p, _sz, _p, _p, _p]),
    "kh_moe_set_shared": (C.c_int, [_p, _p, _p, _p]),
    "kh_moe_run": (C.c_int, [_p, _p, _p, _sz, _p]),
    "kh_moe_run_dev": (C.c_int, [_p, _p, _p, _sz, _p]),
    "kh_moe_route": (C.c_int, [_p, _p, _p, _sz, _p, _p, _p]),
    "kh_debug_moe_picks": (C.c_int, [_p, _p, _sz, _p]),
    "kh_mla_attend": (C.c_int, [_p, _p, _sz, _sz, _p, _p, _sz, C.c_float, _p]),
    "kh_mla_attend_dev": (C.c_int, [_p, _sz, _p, _p, _p, _p, _sz, C.c_float, _p]),
    "kh_qcache_open": (C.c_int, [C.c_char_p, C.POINTER(_p)]),
    "kh_qcache_free": (C.c_int, [_p]),
    "kh_qcache_header": (C.c_char_p, [_p]),
    "kh_qcache_count": (C.c_int, [_p, C.POINTER(_sz)]),
    "kh_qcache_name": (C.c_char_p, [_p, _sz]),
    "kh_qcache_info": (C.c_int, [_p, C.c_char_p, C.POINTER(C.c_int), C.POINTER(_sz), C.POINTER(_sz)]),
    "kh_qcache_vector": (C.c_int, [_p, C.c_char_p, _p, _sz]),
    "kh_qcache_weight": (C.c_int, [_p, _p, C.c_char_p, C.POINTER(_p)]),
}


def declared_symbols() -> list[str]:
    return list(_SIGS)


for _name, (_res, _args) in _SIGS.items():
    _f = getattr(lib, _name)
    _f.restype = _res
    _f.argtypes = _args


def _check(rc: int) -> None:
    if rc == OK:
        return
    msg = (lib.kh_last_error() or b"").decode(errors="replace")
    if rc == DECLINED:
        raise Declined(msg)
    raise KvadError(f"status {rc}: {msg}")


def _ptr(a) -> int | None:
    """Host pointer of a contiguous numpy array (None passes NULL)."""
    if a is None:
        return None
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("arrays crossing the ABI must be C-contiguous")
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class Context:
    """kh_ctx: one device, one stream."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        _check(lib.kh_init(device, C.byref(h)))
        self.h = h
        self._objects = weakref.WeakSet()  # live handles made on this context

    def _own(self, obj) -> None:
        self._objects.add(obj)

    def close(self) -> None:
        """kh_free, after every live object made on this context: their frees
        lock the context, so none may outlive it (parked conversations before
        their session, sessions and MoE layers before the weights they name)."""
        if self.h:
            live = list(self._objects)
            for kind in (Parked, Llm, Moe, KvCache, Weight):
                for obj in live:
                    if isinstance(obj, kind):
                        obj.free()
            lib.kh_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream: int | None) -> None:
        _check(lib.kh_set_stream(self.h, stream))

    def synchronize(self) -> None:
        _check(lib.kh_synchronize(self.h))

    def reserve(self, nbytes: int) -> None:
        _check(lib.kh_reserve(self.h, nbytes))


class Weight:
    """kvad's Weight (quant.rs:195-199), held on the device."""

    def __init__(self, ctx: Context, handle: C.c_void_p, keep=None):
        self.ctx = ctx
        self.h = handle
        ctx._own(self)
        rows, cols, prec, nbytes = _sz(), _sz(), C.c_int(), _sz()
        _check(lib.kh_weight_info(handle, C.byref(rows), C.byref(cols), C.byref(prec), C.byref(nbytes)))
        self.rows, self.cols, self.precision, self.bytes = rows.value, cols.value, prec.value, nbytes.value

    @classmethod
    def from_q8(cls, ctx: Context, rows: int, cols: int, scales, qs) -> "Weight":
        scales = _f32(scales)
        qs = np.ascontiguousarray(qs, dtype=np.int8)
        h = C.c_void_p()
        _check(lib.kh_weight_q8(ctx.h, rows, cols, _ptr(scales), _ptr(qs), C.byref(h)))
        return cls(ctx, h)

    @classmethod
    def from_q4(cls, ctx: Context, rows: int, cols: int, scales, qs) -> "Weight":
        scales = _f32(scales)
        qs = np.ascontiguousarray(qs, dtype=np.uint8)
        h = C.c_void_p()
        _check(lib.kh_weight_q4(ctx.h, rows, cols, _ptr(scales), _ptr(qs), C.byref(h)))
        return cls(ctx, h)

    @classmethod
    def from_q4k(cls, ctx: Context, rows: int, cols: int, blocks) -> "Weight":
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        h = C.c_void_p()
        _check(lib.kh_weight_q4k(ctx.h, rows, cols, _ptr(blocks), C.byref(h)))
        return cls(ctx, h)

    @classmethod
    def from_f32(cls, ctx: Context, w) -> "Weight":
        w = _f32(w)
        h = C.c_void_p()
        _check(lib.kh_weight_f32(ctx.h, w.shape[0], w.shape[1], _ptr(w), C.byref(h)))
        return cls(ctx, h)

    @classmethod
    def quantize(cls, ctx: Context, w, precision: int) -> "Weight":
        """Weight::quantize on the device from host f32 [rows, cols]."""
        w = _f32(w)
        h = C.c_void_p()
        _check(lib.kh_weight_quantize(ctx.h, w.shape[0], w.shape[1], _ptr(w), precision, C.byref(h)))
        return cls(ctx, h)

    @classmethod
    def quantize_dev(cls, ctx: Context, rows: int, cols: int, data_ptr: int, precision: int) -> "Weight":
        h = C.c_void_p()
        _check(lib.kh_weight_quantize_dev(ctx.h, rows, cols, data_ptr, precision, C.byref(h)))
        return cls(ctx, h)

    def parts(self):
        """Weight::parts: (scales or None, qs bytes) copied to the host."""
        n = self.rows * self.cols
        if self.precision == Q8:
            qs, sc = np.empty(n, np.int8), np.empty(n // 32, np.float32)
        elif self.precision == Q4:
            qs, sc = np.empty(n // 2, np.uint8), np.empty(n // 32, np.float32)
        elif self.precision == Q4K:
            qs, sc = np.empty(n // 256 * 144, np.uint8), None
        else:
            qs, sc = np.empty(n, np.float32), None
        _check(lib.kh_weight_parts(self.h, _ptr(qs), _ptr(sc)))
        return sc, qs

    def free(self) -> None:
        if self.h:
            lib.kh_weight_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def matvec_bt(self, x, bias=None) -> np.ndarray:
        x = _f32(x)
        assert x.size == self.cols, "matvec_bt shape mismatch"
        b = None if bias is None else _f32(bias)
        y = np.empty(self.rows, np.float32)
        _check(lib.kh_matvec(self.ctx.h, self.h, _ptr(x), _ptr(b), _ptr(y)))
        return y

    def matvec_bt_dev(self, x_ptr: int, y_ptr: int, bias_ptr: int | None = None) -> None:
        _check(lib.kh_matvec_dev(self.ctx.h, self.h, x_ptr, bias_ptr, y_ptr))

    def matvec_bt_dequant(self, x, bias=None) -> np.ndarray:
        """Weight::matvec_bt_dequant (quant.rs:522-589): weights unpacked to
        f32, x unquantised."""
        x = _f32(x)
        assert x.size == self.cols, "matvec_bt_dequant shape mismatch"
        b = None if bias is None else _f32(bias)
        y = np.empty(self.rows, np.float32)
        _check(lib.kh_matvec_dequant(self.ctx.h, self.h, _ptr(x), _ptr(b), _ptr(y)))
        return y

    def matvec_bt_dequant_dev(self, x_ptr: int, y_ptr: int, bias_ptr: int | None = None) -> None:
        _check(lib.kh_matvec_dequant_dev(self.ctx.h, self.h, x_ptr, bias_ptr, y_ptr))

    def matvec_q_dev(self, qs_ptr: int, scales_ptr: int, sums_ptr: int, y_ptr: int,
                     bias_ptr: int | None = None) -> None:
        _check(lib.kh_matvec_q_dev(self.ctx.h, self.h, qs_ptr, scales_ptr, sums_ptr, bias_ptr, y_ptr))

    def matmul_bt(self, xs, m: int, bias=None) -> np.ndarray:
        xs = _f32(xs)
        assert xs.size == m * self.cols, "matmul_bt shape mismatch"
        b = None if bias is None else _f32(bias)
        y = np.empty(m * self.rows, np.float32)
        _check(lib.kh_matmul(self.ctx.h, self.h, _ptr(xs), m, _ptr(b), _ptr(y)))
        return y

    def matmul_bt_dev(self, xs_ptr: int, m: int, y_ptr: int, bias_ptr: int | None = None) -> None:
        _check(lib.kh_matmul_dev(self.ctx.h, self.h, xs_ptr, m, bias_ptr, y_ptr))

    def row(self, r: int) -> np.ndarray:
        out = np.empty(self.cols, np.float32)
        _check(lib.kh_weight_row(self.ctx.h, self.h, r, _ptr(out)))
        return out

    def block_dots(self, x) -> np.ndarray:
        x = _f32(x)
        d = np.empty(self.rows * (self.cols // 32), np.int32)
        _check(lib.kh_debug_block_dots(self.ctx.h, self.h, _ptr(x), _ptr(d)))
        return d.reshape(self.rows, self.cols // 32)


def matvec_many(ctx: Context, jobs) -> list[np.ndarray] | None:
    """quant::matvec_many: None when a weight is f32, as the reference does."""
    n = len(jobs)
    xs = [_f32(x) for _, x in jobs]
    # the same array object twice in a row is the same input, as in Rust
    for i in range(1, n):
        if jobs[i][1] is jobs[i - 1][1]:
            xs[i] = xs[i - 1]
    ys = [np.empty(w.rows, np.float32) for w, _ in jobs]
    W = (C.c_void_p * n)(*[w.h.value for w, _ in jobs])
    X = (C.c_void_p * n)(*[_ptr(x) for x in xs])
    Y = (C.c_void_p * n)(*[_ptr(y) for y in ys])
    rc = lib.kh_matvec_many(ctx.h, n, W, X, Y)
    if rc == DECLINED:
        return None
    _check(rc)
    return ys


def stream_dev(ctx: Context, weights, sink_ptr: int) -> None:
    """kh_debug_stream_dev: one launch reading the weights' bytes once (a timing aid)."""
    arr = (C.c_void_p * len(weights))(*[w.h.value for w in weights])
    _check(lib.kh_debug_stream_dev(ctx.h, len(weights), arr, C.c_void_p(sink_ptr)))


def qact_dev(ctx: Context, x_ptr: int, m: int, n: int, qs_ptr: int, scales_ptr: int, sums_ptr: int) -> None:
    """QActBatch::new on device pointers."""
    _check(lib.kh_qact_dev(ctx.h, x_ptr, m, n, qs_ptr, scales_ptr, sums_ptr))


def qact(ctx: Context, x):
    """QActivation::new on the device: (qs, scales, sums)."""
    x = _f32(x)
    n = x.size
    qs = np.empty(n, np.int8)
    sc = np.empty(n // 32, np.float32)
    su = np.empty(n // 32, np.int32)
    _check(lib.kh_debug_qact(ctx.h, _ptr(x), n, _ptr(qs), _ptr(sc), _ptr(su)))
    return qs, sc, su


def quant_check(ctx: Context):
    """The activation quantiser's arithmetic over every float (a self-check):
    (scales, inverses, codes) that differ from IEEE division and Rust's
    rounding; all zero on a correct build."""
    counts = np.zeros(3, np.uint64)
    _check(lib.kh_debug_quant_check(ctx.h, _ptr(counts)))
    return tuple(int(c) for c in counts)


class QCache:
    """The quantised-weight cache file (crates/llm/src/qcache.rs): the
    container mapped and its tensor table parsed (Container::open,
    parse_entry); `weight` uploads an entry as a device Weight
    (Mapped::build), `vector` copies an f32 vector to the host
    (Mapped::vector).  Opening needs no device."""

    def __init__(self, path):
        h = C.c_void_p()
        _check(lib.kh_qcache_open(str(path).encode(), C.byref(h)))
        self.h = h

    def close(self) -> None:
        if self.h:
            lib.kh_qcache_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def header(self) -> str:
        return lib.kh_qcache_header(self.h).decode()

    def names(self) -> list[str]:
        n = C.c_size_t()
        _check(lib.kh_qcache_count(self.h, C.byref(n)))
        return [lib.kh_qcache_name(self.h, i).decode() for i in range(n.value)]

    def info(self, name: str) -> tuple[int, int, int]:
        """(precision, rows, cols) of the device weight the entry becomes."""
        prec, rows, cols = C.c_int(), C.c_size_t(), C.c_size_t()
        _check(lib.kh_qcache_info(self.h, name.encode(), C.byref(prec), C.byref(rows), C.byref(cols)))
        return prec.value, rows.value, cols.value

    def vector(self, name: str) -> np.ndarray:
        _, rows, cols = self.info(name)
        out = np.empty(cols, np.float32)
        _check(lib.kh_qcache_vector(self.h, name.encode(), _ptr(out), cols))
        return out

    def weight(self, ctx: "Context", name: str) -> "Weight":
        h = C.c_void_p()
        _check(lib.kh_qcache_weight(ctx.h, self.h, name.encode(), C.byref(h)))
        return Weight(ctx, h)


@dataclass(frozen=True)
class Spec:
    """The attention geometry of model::Spec (model/mod.rs:298-312)."""

    n_head: int
    n_kv_head: int
    head_dim: int

    @property
    def kv_dim(self) -> int:
        return self.n_kv_head * self.head_dim

    @property
    def group_size(self) -> int:
        return self.n_head // self.n_kv_head


class KvCache:
    """KvCache (model/mod.rs:612-749) with device-resident layers."""

    def __init__(self, ctx: Context, n_layer: int, k_dim: int, v_dim: int, capacity: int = 0):
        h = C.c_void_p()
        _check(lib.kh_kv_new(ctx.h, n_layer, k_dim, v_dim, capacity, C.byref(h)))
        self.ctx, self.h = ctx, h
        ctx._own(self)
        self.n_layer, self.k_dim, self.v_dim = n_layer, k_dim, v_dim

    def free(self) -> None:
        if self.h:
            lib.kh_kv_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def push(self, layer: int, k, v) -> None:
        k, v = _f32(k), _f32(v)
        m = k.size // self.k_dim
        assert k.size == m * self.k_dim and v.size == m * self.v_dim
        _check(lib.kh_kv_push(self.h, layer, _ptr(k), _ptr(v), m))

    def push_dev(self, layer: int, k_ptr: int, v_ptr: int, m: int) -> None:
        _check(lib.kh_kv_push_dev(self.h, layer, k_ptr, v_ptr, m))

    @property
    def len(self) -> int:
        n = _sz()
        _check(lib.kh_kv_len(self.h, C.byref(n)))
        return n.value

    @len.setter
    def len(self, value: int) -> None:
        _check(lib.kh_kv_set_len(self.h, value))

    def truncate(self, n: int) -> int:
        kept = _sz()
        _check(lib.kh_kv_truncate(self.h, n, C.byref(kept)))
        return kept.value

    def clear(self) -> None:
        _check(lib.kh_kv_clear(self.h))

    def _read(self, fn, layer: int, dim: int) -> np.ndarray:
        rows = _sz()
        _check(fn(self.h, layer, None, C.byref(rows)))
        out = np.empty(rows.value * dim, np.float32)
        _check(fn(self.h, layer, _ptr(out) if out.size else None, C.byref(rows)))
        return out

    def keys(self, layer: int) -> np.ndarray:
        return self._read(lib.kh_kv_keys, layer, self.k_dim)

    def values(self, layer: int) -> np.ndarray:
        return self._read(lib.kh_kv_values, layer, self.v_dim)

    def layer_ptrs(self, layer: int) -> tuple[int, int]:
        k, v = C.c_void_p(), C.c_void_p()
        _check(lib.kh_kv_layer_ptrs(self.h, layer, C.byref(k), C.byref(v)))
        return k.value, v.value


def attend(ctx: Context, spec: Spec, q, cache: KvCache, layer: int, n_positions: int) -> np.ndarray:
    """model::attend over a device cache layer."""
    q = _f32(q)
    out = np.empty(spec.n_head * spec.head_dim, np.float32)
    _check(lib.kh_attend(ctx.h, cache.h, layer, spec.n_head, spec.n_kv_head, spec.head_dim, _ptr(q),
                         n_positions, _ptr(out)))
    return out


def mla_attend(ctx: Context, cache: "KvCache", layer: int, n_head: int, q_lat, q_pe, n_positions: int,
               scale: float) -> np.ndarray:
    """The latent-attention core of DeepSeek's Model::attend (model/deepseek.rs:553-591)
    over a cache whose keys are the rope rows (64) and values the latents (512)."""
    ql, qp = _f32(q_lat), _f32(q_pe)
    assert ql.size == n_head * 512 and qp.size == n_head * 64
    out = np.empty(n_head * 512, np.float32)
    _check(lib.kh_mla_attend(ctx.h, cache.h, layer, n_head, _ptr(ql), _ptr(qp), n_positions, scale, _ptr(out)))
    return out


def mla_attend_dev(ctx: Context, n_head: int, q_lat_ptr: int, q_pe_ptr: int, c_ptr: int, pe_ptr: int,
                   n_positions: int, scale: float, out_ptr: int) -> None:
    _check(lib.kh_mla_attend_dev(ctx.h, n_head, q_lat_ptr, q_pe_ptr, c_ptr, pe_ptr, n_positions, scale, out_ptr))


def attend_dev(ctx: Context, spec: Spec, q_ptr: int, k_ptr: int, v_ptr: int, n_positions: int,
               out_ptr: int) -> None:
    _check(lib.kh_attend_dev(ctx.h, spec.n_head, spec.n_kv_head, spec.head_dim, q_ptr, k_ptr, v_ptr,
                             n_positions, out_ptr))


class Moe:
    """kvad's Moe (model/ffn.rs:474-708) on the device: a router and n_experts
    SwiGLU experts (plus an optional shared expert).  The Weight objects are
    kept referenced here, since the layer borrows their device arrays."""

    def __init__(self, ctx: Context, n_experts: int, top_k: int, hidden: int, inter: int, scoring: int = SOFTMAX,
                 select: int = GREEDY, n_group: int = 1, topk_group: int = 1, norm_topk: bool = False,
                 scale: float = 1.0, bias=None):
        self.ctx, self.n_experts, self.top_k, self.hidden, self.inter = ctx, n_experts, top_k, hidden, inter
        b = None if bias is None else _f32(bias)
        self.h = C.c_void_p()
        _check(lib.kh_moe_new(ctx.h, n_experts, top_k, hidden, inter, scoring, select, n_group, topk_group,
                              int(norm_topk), scale, _ptr(b), C.byref(self.h)))
        ctx._own(self)
        self._keep = {}

    def set_router(self, w: Weight) -> None:
        _check(lib.kh_moe_set_router(self.h, w.h))
        self._keep["router"] = w

    def set_expert(self, x: int, gate: Weight, up: Weight, down: Weight) -> None:
        _check(lib.kh_moe_set_expert(self.h, x, gate.h, up.h, down.h))
        self._keep[x] = (gate, up, down)

    def set_shared(self, gate: Weight, up: Weight, down: Weight) -> None:
        _check(lib.kh_moe_set_shared(self.h, gate.h, up.h, down.h))
        self._keep["shared"] = (gate, up, down)

    def run(self, hs, m: int) -> np.ndarray:
        """Moe::run: out [m * hidden] for hs [m * hidden]."""
        hs = _f32(hs)
        assert hs.size == m * self.hidden, "moe shape mismatch"
        out = np.empty(m * self.hidden, np.float32)
        _check(lib.kh_moe_run(self.ctx.h, self.h, _ptr(hs), m, _ptr(out)))
        return out

    def run_dev(self, hs_ptr: int, m: int, out_ptr: int) -> None:
        _check(lib.kh_moe_run_dev(self.ctx.h, self.h, hs_ptr, m, out_ptr))

    def route(self, logits, m: int):
        """Router::route per token: a list of [(expert, weight), ...] in pick order."""
        logits = _f32(logits)
        e = np.empty(m * self.top_k, np.int32)
        w = np.empty(m * self.top_k, np.float32)
        c = np.empty(m, np.int32)
        _check(lib.kh_moe_route(self.ctx.h, self.h, _ptr(logits), m, _ptr(e), _ptr(w), _ptr(c)))
        k = self.top_k
        return [[(int(e[i * k + j]), float(w[i * k + j])) for j in range(int(c[i]))] for i in range(m)]

    def picks(self, m: int, hidden_codes: bool = False) -> dict:
        """The last run's intermediates (kh_debug_moe_picks) for its m tokens,
        picks in expert order: logits, count, experts, weights, gate, up,
        out (each expert's down projection), shared_gate/_up/_out when a
        shared expert is set, hidden_qs/_scales (m > 1) when asked."""
        k, inter, hid = self.top_k, self.inter, self.hidden
        r = {"logits": np.zeros((m, self.n_experts), np.float32), "count": np.zeros(m, np.int32),
             "experts": np.zeros((m, k), np.int32), "weights": np.zeros((m, k), np.float32),
             "gate": np.zeros((m, k, inter), np.float32), "up": np.zeros((m, k, inter), np.float32),
             "out": np.zeros((m, k, hid), np.float32)}
        if hidden_codes:
            r["hidden_qs"] = np.zeros((m, k, inter), np.int8)
            r["hidden_scales"] = np.zeros((m, k, inter // 32), np.float32)
        if "shared" in self._keep:
            sh = self._keep["shared"][0].rows
            r["shared_gate"], r["shared_up"] = np.zeros((m, sh), np.float32), np.zeros((m, sh), np.float32)
            r["shared_out"] = np.zeros((m, hid), np.float32)
        names = ["logits", "count", "experts", "weights", "gate", "up", "hidden_qs", "hidden_scales", "out",
                 "shared_gate", "shared_up", "shared_out"]
        ptrs = (_p * len(names))(*[r[n].ctypes.data if n in r else None for n in names])
        _check(lib.kh_debug_moe_picks(self.ctx.h, self.h, m, ptrs))
        return r

    def free(self) -> None:
        if self.h:
            lib.kh_moe_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---- decode glue on device pointers (tensor.rs:297-472) ----------------------

def rms_norm_dev(ctx: Context, x_ptr: int, w_ptr: int, m: int, n: int, eps: float, out_ptr: int) -> None:
    _check(lib.kh_rms_norm_dev(ctx.h, x_ptr, w_ptr, m, n, eps, out_ptr))


def rope_dev(ctx: Context, cos_ptr: int, sin_ptr: int, half: int, x_ptr: int, m: int, n_vec: int, pos0: int,
             interleaved: bool = False) -> None:
    _check(lib.kh_rope_dev(ctx.h, cos_ptr, sin_ptr, half, x_ptr, m, n_vec, pos0, int(interleaved)))


def swiglu_dev(ctx: Context, gate_ptr: int, up_ptr: int, n: int) -> None:
    _check(lib.kh_swiglu_dev(ctx.h, gate_ptr, up_ptr, n))


def softmax_dev(ctx: Context, x_ptr: int, m: int, n: int) -> None:
    _check(lib.kh_softmax_dev(ctx.h, x_ptr, m, n))


class LlmSpec(C.Structure):
    """kh_llm_spec: a Llama-family decoder's sizes (model/mod.rs:286-330)."""
    _fields_ = [(n, C.c_size_t) for n in ("n_layer", "n_embd", "n_head", "n_kv_head", "head_dim", "n_ff", "vocab",
                                         "n_ctx")] + [("eps", C.c_float), ("rope_interleaved", C.c_int)]


class Llm:
    """A device-resident decoder session (the Session trait's device backend,
    model/mod.rs:839-976) over borrowed Weight handles (kept referenced here)."""

    def __init__(self, ctx: Context, **spec):
        self.ctx = ctx
        self.spec = LlmSpec(**spec)
        self.h = C.c_void_p()
        _check(lib.kh_llm_new(ctx.h, C.byref(self.spec), C.byref(self.h)))
        ctx._own(self)
        self._keep = {}

    def set_layer(self, l: int, q, k, v, o, gate, up, down, attn_norm, mlp_norm, q_b=None, k_b=None, v_b=None,
                  q_norm=None, k_norm=None) -> None:
        vec = [None if a is None else _f32(a) for a in (attn_norm, mlp_norm, q_b, k_b, v_b, q_norm, k_norm)]
        _check(lib.kh_llm_set_layer(self.h, l, q.h, k.h, v.h, o.h, gate.h, up.h, down.h, *[_ptr(a) for a in vec]))
        self._keep[l] = (q, k, v, o, gate, up, down)

    def set_ends(self, embed, final_norm, lm_head=None) -> None:
        fn = _f32(final_norm)
        _check(lib.kh_llm_set_ends(self.h, embed.h, _ptr(fn), None if lm_head is None else lm_head.h))
        self._keep["ends"] = (embed, lm_head)

    def set_rope(self, cos_t, sin_t, max_pos: int) -> None:
        c, s = _f32(cos_t), _f32(sin_t)
        _check(lib.kh_llm_set_rope(self.h, _ptr(c), _ptr(s), max_pos))

    def forward(self, token: int, want_logits: bool = True):
        """(logits or None, next token) for one token at the next position."""
        logits = np.empty(self.spec.vocab, np.float32) if want_logits else None
        nxt = C.c_int32()
        _check(lib.kh_llm_forward(self.ctx.h, self.h, token, _ptr(logits), C.byref(nxt)))
        return logits, nxt.value

    def trace(self, token: int) -> dict:
        """forward() of one token with each sub-block's results copied out
        (kh_debug_llm_trace): x_embed, and per layer qkv, k_cache, v_cache
        (the positions held after the push), att, x_attn, gate, up, x_mlp;
        then logits."""
        s = self.spec
        L, n = s.n_layer, len(self) + 1
        qd, kvd = s.n_head * s.head_dim, s.n_kv_head * s.head_dim
        r = {"x_embed": np.zeros(s.n_embd, np.float32), "qkv": np.zeros((L, qd + 2 * kvd), np.float32),
             "k_cache": np.zeros((L, n, kvd), np.float32), "v_cache": np.zeros((L, n, kvd), np.float32),
             "att": np.zeros((L, qd), np.float32), "x_attn": np.zeros((L, s.n_embd), np.float32),
             "gate": np.zeros((L, s.n_ff), np.float32), "up": np.zeros((L, s.n_ff), np.float32),
             "x_mlp": np.zeros((L, s.n_embd), np.float32), "logits": np.zeros(s.vocab, np.float32)}
        names = ["x_embed", "qkv", "k_cache", "v_cache", "att", "x_attn", "gate", "up", "x_mlp", "logits"]
        ptrs = (_p * len(names))(*[r[k].ctypes.data for k in names])
        _check(lib.kh_debug_llm_trace(self.ctx.h, self.h, token, ptrs))
        return r

    def forward_tokens(self, tokens, want_logits: bool = True):
        """Session::forward(&[u32]) (model/mod.rs:842): the tokens at the next
        positions, read in passes cut where prefill_pass says; (logits of the
        last token or None, its greedy next token)."""
        toks = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty(self.spec.vocab, np.float32) if want_logits else None
        nxt = C.c_int32()
        _check(lib.kh_llm_forward_tokens(self.ctx.h, self.h, _ptr(toks), toks.size, _ptr(logits), C.byref(nxt)))
        return logits, nxt.value

    def prefill_pass(self, left: int) -> int:
        """Session::prefill_pass (model/mod.rs:866): tokens of `left` the next pass reads."""
        n = _sz()
        _check(lib.kh_llm_prefill_pass(self.h, left, C.byref(n)))
        return n.value

    def reading(self, chunk: int) -> "Llm":
        """CpuSession::reading (model/mod.rs:1079): `chunk` prompt tokens a pass (0: the default)."""
        _check(lib.kh_llm_set_prefill_chunk(self.h, chunk))
        return self

    def trace_pass(self, tokens) -> dict:
        """One pass of the tokens on the rows path with each sub-block's rows
        copied out (kh_debug_llm_trace_pass): x_embed [n, e]; per layer qkv
        [n, qd + 2 kvd], k_cache / v_cache (every position held after the
        pass), att, x_attn, gate, up, x_mlp; logits of the last row."""
        toks = np.ascontiguousarray(tokens, np.int32)
        s = self.spec
        L, n, held = s.n_layer, toks.size, len(self) + toks.size
        qd, kvd = s.n_head * s.head_dim, s.n_kv_head * s.head_dim
        r = {"x_embed": np.zeros((n, s.n_embd), np.float32), "qkv": np.zeros((L, n, qd + 2 * kvd), np.float32),
             "k_cache": np.zeros((L, held, kvd), np.float32), "v_cache": np.zeros((L, held, kvd), np.float32),
             "att": np.zeros((L, n, qd), np.float32), "x_attn": np.zeros((L, n, s.n_embd), np.float32),
             "gate": np.zeros((L, n, s.n_ff), np.float32), "up": np.zeros((L, n, s.n_ff), np.float32),
             "x_mlp": np.zeros((L, n, s.n_embd), np.float32), "logits": np.zeros(s.vocab, np.float32)}
        names = ["x_embed", "qkv", "k_cache", "v_cache", "att", "x_attn", "gate", "up", "x_mlp", "logits"]
        ptrs = (_p * len(names))(*[r[k].ctypes.data for k in names])
        _check(lib.kh_debug_llm_trace_pass(self.ctx.h, self.h, _ptr(toks), n, ptrs))
        return r

    def generate(self, token: int, n: int) -> np.ndarray:
        out = np.empty(n, np.int32)
        _check(lib.kh_llm_generate(self.ctx.h, self.h, token, n, _ptr(out)))
        return out

    def generate_launch(self, n: int) -> None:
        _check(lib.kh_llm_generate_launch(self.ctx.h, self.h, n))

    def __len__(self) -> int:
        n = _sz()
        _check(lib.kh_llm_len(self.h, C.byref(n)))
        return n.value

    def truncate(self, n: int) -> None:
        _check(lib.kh_llm_truncate(self.h, n))

    def park(self) -> "Parked":
        """Session::park (model/mod.rs:883-893): the conversation held so
        far, set aside; the session is left with an empty one."""
        h = C.c_void_p()
        _check(lib.kh_llm_park(self.h, C.byref(h)))
        return Parked(h, self.ctx)

    def resume(self, parked: "Parked") -> None:
        """Session::resume (model/mod.rs:895-897): `parked` back in place of
        the conversation held, which is dropped.  Consumes `parked`."""
        h, parked.h = parked.h, None
        _check(lib.kh_llm_resume(self.h, h))

    def forward_each(self, tokens, caches, want_logits: bool = True):
        """Session::forward_each (model/mod.rs:899-930, llama.rs:418-434):
        tokens[i] onto caches[i], all in one pass; (logits [n, vocab] or
        None, next tokens [n])."""
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        n = toks.size
        if n != len(caches):
            raise KvadError("a token for each conversation, and a conversation for each token")
        arr = (C.c_void_p * max(n, 1))(*[c.h for c in caches])
        logits = np.empty((n, self.spec.vocab), np.float32) if want_logits else None
        nxt = np.empty(n, np.int32)
        _check(lib.kh_llm_forward_each(self.ctx.h, self.h, n, _ptr(toks), C.cast(arr, C.c_void_p), _ptr(logits),
                                       _ptr(nxt)))
        return logits, nxt

    def free(self) -> None:
        if self.h:
            lib.kh_llm_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Parked:
    """A conversation set aside by Llm.park (the Session trait's Parked,
    model/mod.rs:837): its device cache and length."""

    def __init__(self, h, ctx: Context | None = None):
        self.h = h
        if ctx is not None:
            ctx._own(self)

    def __len__(self) -> int:
        n = _sz()
        _check(lib.kh_llm_parked_len(self.h, C.byref(n)))
        return n.value

    def free(self) -> None:
        if self.h:
            lib.kh_llm_parked_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

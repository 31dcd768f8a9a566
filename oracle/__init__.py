"""Python wrapper of the CPU oracle (oracle/kvad_oracle.c).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, and only as the checker or the CPU baseline --
never as the path being measured or shipped.

Each function restates the reference line for line; the C source cites the
lines.  Arrays are numpy, shapes as in the reference.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libkvad_oracle.so"
LIB_NATIVE = HERE / "libkvad_oracle_native.so"


def build() -> None:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "-B"], check=True)


def _load(path: Path) -> C.CDLL:
    if not path.exists():
        build()
    return C.CDLL(str(path))


_p = C.c_void_p
_sz = C.c_size_t
_f = C.c_float


def _declare(lib: C.CDLL) -> C.CDLL:
    sigs = {
        "kvo_fill_normal": (None, [C.c_uint64, _f, _p, _sz]),
        "kvo_set_threads": (None, [C.c_int]),
        "kvo_get_threads": (C.c_int, []),
        "kvo_quantize_q8": (None, [_p, _sz, _sz, _p, _p]),
        "kvo_quantize_q4": (None, [_p, _sz, _sz, _p, _p]),
        "kvo_qact": (None, [_p, _sz, _p, _p, _p]),
        "kvo_qact_batch": (None, [_p, _sz, _sz, _p, _p, _p]),
        "kvo_f32_to_f16": (C.c_uint16, [_f]),
        "kvo_f16_to_f32": (_f, [C.c_uint16]),
        "kvo_quantize_q4k": (None, [_p, _sz, _sz, _p]),
        "kvo_row_q8": (None, [_p, _p, _sz, _sz, _p]),
        "kvo_row_q4": (None, [_p, _p, _sz, _sz, _p]),
        "kvo_row_q4k": (None, [_p, _sz, _sz, _p]),
        "kvo_block_dots_q8": (None, [_p, _sz, _sz, _p, _p]),
        "kvo_block_dots_q4": (None, [_p, _sz, _sz, _p, _p, _p]),
        "kvo_block_dots_q4k": (None, [_p, _sz, _sz, _p, _p]),
        "kvo_matvec_q8": (None, [_p, _p, _sz, _sz, _p, _p, _p]),
        "kvo_matvec_q4": (None, [_p, _p, _sz, _sz, _p, _p, _p]),
        "kvo_matvec_q4k": (None, [_p, _sz, _sz, _p, _p, _p]),
        "kvo_matvec_q4k_fast": (None, [_p, _sz, _sz, _p, _p, _p]),
        "kvo_matvec_f32": (None, [_p, _sz, _sz, _p, _p, _p]),
        "kvo_matvec_dequant": (None, [C.c_int, _p, _p, _sz, _sz, _p, _p]),
        "kvo_matmul_q8": (None, [_p, _p, _sz, _sz, _p, _sz, _p, _p]),
        "kvo_matmul_q4": (None, [_p, _p, _sz, _sz, _p, _sz, _p, _p]),
        "kvo_matmul_q4k": (None, [_p, _sz, _sz, _p, _sz, _p, _p]),
        "kvo_gemm_f32": (None, [_p, _sz, _p, _sz, _sz, _p]),
        "kvo_matmul_f32": (None, [_p, _sz, _sz, _p, _sz, _p, _p]),
        "kvo_dot": (_f, [_p, _p, _sz]),
        "kvo_softmax": (None, [_p, _sz]),
        "kvo_rms_norm": (None, [_p, _p, _sz, _f, _p]),
        "kvo_swiglu": (None, [_p, _p, _sz]),
        "kvo_rope_tables": (None, [_sz, _sz, _f, _p, _p]),
        "kvo_rope_apply": (None, [_p, _p, _sz, _p, _sz]),
        "kvo_rope_apply_interleaved": (None, [_p, _p, _sz, _p, _sz]),
        "kvo_attend": (None, [_sz, _sz, _sz, _p, _p, _p, _sz, _p]),
        "kvo_mla_attend": (None, [_sz, _sz, _sz, _p, _p, _p, _p, _sz, C.c_float, _p]),
        "kvo_route": (C.c_int, [_p, _sz, _sz, C.c_int, C.c_int, _sz, _sz, C.c_int, _f, _p, _p, _p]),
        "kvo_moe_run_q8": (None, [_p, _sz, _sz, _sz, _sz, _sz, C.c_int, C.c_int, _sz, _sz, C.c_int, _f, _p]
                           + [_p] * 8 + [_sz] + [_p] * 7),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _declare(_load(LIB))
_native = None


def native_lib() -> C.CDLL:
    """The -march=native build, for the second CPU-baseline column."""
    global _native
    if _native is None:
        _native = _declare(_load(LIB_NATIVE))
    return _native


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def P(a):
    return None if a is None else a.ctypes.data


def set_threads(n: int) -> None:
    lib.kvo_set_threads(n)
    if _native is not None:
        _native.kvo_set_threads(n)


def threads() -> int:
    return lib.kvo_get_threads()


# ---- seeded inputs --------------------------------------------------------

def normal(seed: int, n: int, scale: float = 1.0) -> np.ndarray:
    """n values of nervus Rng(seed).normal() * scale (crates/nervus/src/rng.rs:35-39)."""
    out = np.empty(n, np.float32)
    lib.kvo_fill_normal(seed, scale, P(out), n)
    return out


# ---- quantisation ---------------------------------------------------------

def quantize_q8(w, rows: int, cols: int):
    w = _c(w, np.float32)
    s = np.empty(rows * cols // 32, np.float32)
    q = np.empty(rows * cols, np.int8)
    lib.kvo_quantize_q8(P(w), rows, cols, P(s), P(q))
    return s, q


def quantize_q4(w, rows: int, cols: int):
    w = _c(w, np.float32)
    s = np.empty(rows * cols // 32, np.float32)
    q = np.empty(rows * cols // 2, np.uint8)
    lib.kvo_quantize_q4(P(w), rows, cols, P(s), P(q))
    return s, q


def quantize_q4k(w, rows: int, cols: int) -> np.ndarray:
    w = _c(w, np.float32)
    b = np.empty(rows * cols // 256 * 144, np.uint8)
    lib.kvo_quantize_q4k(P(w), rows, cols, P(b))
    return b


def qact(x):
    x = _c(x, np.float32)
    n = x.size
    q = np.empty(n, np.int8)
    s = np.empty(n // 32, np.float32)
    su = np.empty(n // 32, np.int32)
    lib.kvo_qact(P(x), n, P(q), P(s), P(su))
    return q, s, su


def f32_to_f16(x: float) -> int:
    return lib.kvo_f32_to_f16(x)


def f16_to_f32(h: int) -> float:
    return lib.kvo_f16_to_f32(h)


# ---- rows and dots --------------------------------------------------------

def row_q8(scales, qs, cols: int, r: int) -> np.ndarray:
    out = np.empty(cols, np.float32)
    lib.kvo_row_q8(P(_c(scales, np.float32)), P(_c(qs, np.int8)), cols, r, P(out))
    return out


def row_q4(scales, qs, cols: int, r: int) -> np.ndarray:
    out = np.empty(cols, np.float32)
    lib.kvo_row_q4(P(_c(scales, np.float32)), P(_c(qs, np.uint8)), cols, r, P(out))
    return out


def row_q4k(blocks, cols: int, r: int) -> np.ndarray:
    out = np.empty(cols, np.float32)
    lib.kvo_row_q4k(P(_c(blocks, np.uint8)), cols, r, P(out))
    return out


def block_dots_q8(qs, rows: int, cols: int, xq) -> np.ndarray:
    d = np.empty(rows * cols // 32, np.int32)
    lib.kvo_block_dots_q8(P(_c(qs, np.int8)), rows, cols, P(_c(xq, np.int8)), P(d))
    return d.reshape(rows, cols // 32)


def block_dots_q4(qs, rows: int, cols: int, xq, xsums) -> np.ndarray:
    d = np.empty(rows * cols // 32, np.int32)
    lib.kvo_block_dots_q4(P(_c(qs, np.uint8)), rows, cols, P(_c(xq, np.int8)), P(_c(xsums, np.int32)), P(d))
    return d.reshape(rows, cols // 32)


def block_dots_q4k(blocks, rows: int, cols: int, xq) -> np.ndarray:
    d = np.empty(rows * cols // 32, np.int32)
    lib.kvo_block_dots_q4k(P(_c(blocks, np.uint8)), rows, cols, P(_c(xq, np.int8)), P(d))
    return d.reshape(rows, cols // 32)


# ---- GEMV / GEMM ----------------------------------------------------------

def matvec_q8(scales, qs, rows, cols, x, bias=None, L=None) -> np.ndarray:
    L = L or lib
    y = np.empty(rows, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    L.kvo_matvec_q8(P(_c(scales, np.float32)), P(_c(qs, np.int8)), rows, cols, P(_c(x, np.float32)), P(b), P(y))
    return y


def matvec_q4(scales, qs, rows, cols, x, bias=None, L=None) -> np.ndarray:
    L = L or lib
    y = np.empty(rows, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    L.kvo_matvec_q4(P(_c(scales, np.float32)), P(_c(qs, np.uint8)), rows, cols, P(_c(x, np.float32)), P(b), P(y))
    return y


def matvec_q4k(blocks, rows, cols, x, bias=None, L=None) -> np.ndarray:
    L = L or lib
    y = np.empty(rows, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    L.kvo_matvec_q4k(P(_c(blocks, np.uint8)), rows, cols, P(_c(x, np.float32)), P(b), P(y))
    return y


def matvec_q4k_fast(blocks, rows, cols, x, bias=None, L=None) -> np.ndarray:
    """matvec_q4k organised for the CPU baseline (equal to the bit)."""
    L = L or lib
    y = np.empty(rows, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    L.kvo_matvec_q4k_fast(P(_c(blocks, np.uint8)), rows, cols, P(_c(x, np.float32)), P(b), P(y))
    return y


def matvec_f32(w, rows, cols, x, bias=None) -> np.ndarray:
    y = np.empty(rows, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    lib.kvo_matvec_f32(P(_c(w, np.float32)), rows, cols, P(_c(x, np.float32)), P(b), P(y))
    return y


def matvec_dequant(precision: int, scales, qs, rows, cols, x) -> np.ndarray:
    y = np.empty(rows, np.float32)
    qs = _c(qs, np.int8 if precision == 1 else np.uint8)
    lib.kvo_matvec_dequant(precision, P(_c(scales, np.float32)), P(qs), rows, cols, P(_c(x, np.float32)), P(y))
    return y


def matmul_q8(scales, qs, rows, cols, xs, m, bias=None, L=None) -> np.ndarray:
    L = L or lib
    y = np.empty(m * rows, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    L.kvo_matmul_q8(P(_c(scales, np.float32)), P(_c(qs, np.int8)), rows, cols, P(_c(xs, np.float32)), m, P(b), P(y))
    return y


def matmul_q4(scales, qs, rows, cols, xs, m, bias=None, L=None) -> np.ndarray:
    L = L or lib
    y = np.empty(m * rows, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    L.kvo_matmul_q4(P(_c(scales, np.float32)), P(_c(qs, np.uint8)), rows, cols, P(_c(xs, np.float32)), m, P(b), P(y))
    return y


def matmul_q4k(blocks, rows, cols, xs, m, bias=None, L=None) -> np.ndarray:
    L = L or lib
    y = np.empty(m * rows, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    L.kvo_matmul_q4k(P(_c(blocks, np.uint8)), rows, cols, P(_c(xs, np.float32)), m, P(b), P(y))
    return y


def gemm_f32(xs, m, w, rows, cols) -> np.ndarray:
    out_t = np.empty(rows * m, np.float32)
    lib.kvo_gemm_f32(P(_c(xs, np.float32)), m, P(_c(w, np.float32)), rows, cols, P(out_t))
    return out_t


def matmul_f32(w, rows, cols, xs, m, bias=None, L=None) -> np.ndarray:
    L = L or lib
    y = np.empty(m * rows, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    L.kvo_matmul_f32(P(_c(w, np.float32)), rows, cols, P(_c(xs, np.float32)), m, P(b), P(y))
    return y


# ---- small pieces ---------------------------------------------------------

def dot(a, b) -> float:
    a, b = _c(a, np.float32), _c(b, np.float32)
    return lib.kvo_dot(P(a), P(b), a.size)


def softmax(x) -> np.ndarray:
    x = _c(x, np.float32).copy()
    lib.kvo_softmax(P(x), x.size)
    return x


def rms_norm(x, w, eps: float) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib.kvo_rms_norm(P(x), P(_c(w, np.float32)), x.size, eps, P(out))
    return out


def swiglu(gate, up) -> np.ndarray:
    g = _c(gate, np.float32).copy()
    lib.kvo_swiglu(P(g), P(_c(up, np.float32)), g.size)
    return g


def rope_tables(head_dim: int, max_pos: int, theta: float):
    half = head_dim // 2
    c = np.empty(max_pos * half, np.float32)
    s = np.empty(max_pos * half, np.float32)
    lib.kvo_rope_tables(head_dim, max_pos, theta, P(c), P(s))
    return c, s


def rope_apply(cos_t, sin_t, half: int, x, pos: int) -> np.ndarray:
    x = _c(x, np.float32).copy()
    lib.kvo_rope_apply(P(cos_t), P(sin_t), half, P(x), pos)
    return x


def rope_apply_interleaved(cos_t, sin_t, half: int, x, pos: int) -> np.ndarray:
    x = _c(x, np.float32).copy()
    lib.kvo_rope_apply_interleaved(P(cos_t), P(sin_t), half, P(x), pos)
    return x


def attend(n_head, n_kv_head, head_dim, q, k_cache, v_cache, n_positions, L=None) -> np.ndarray:
    L = L or lib
    out = np.empty(n_head * head_dim, np.float32)
    L.kvo_attend(n_head, n_kv_head, head_dim, P(_c(q, np.float32)), P(_c(k_cache, np.float32)),
                 P(_c(v_cache, np.float32)), n_positions, P(out))
    return out


def mla_attend(n_head, lat, rope, q_lat, q_pe, c_cache, pe_cache, n_positions, scale, L=None) -> np.ndarray:
    L = L or lib
    out = np.empty(n_head * lat, np.float32)
    L.kvo_mla_attend(n_head, lat, rope, P(_c(q_lat, np.float32)), P(_c(q_pe, np.float32)),
                     P(_c(c_cache, np.float32)), P(_c(pe_cache, np.float32)), n_positions, scale, P(out))
    return out


def route(logits, top_k: int, scoring: int = 0, select: int = 0, n_group: int = 1, topk_group: int = 1,
          norm_topk: bool = False, scale: float = 1.0, bias=None):
    """Router::route: list of (expert, weight) in pick order."""
    logits = _c(logits, np.float32)
    n = logits.size
    e = np.empty(max(top_k, 1), np.int32)
    w = np.empty(max(top_k, 1), np.float32)
    b = None if bias is None else _c(bias, np.float32)
    got = lib.kvo_route(P(logits), n, top_k, scoring, select, n_group, topk_group, int(norm_topk), scale, P(b),
                        P(e), P(w))
    return [(int(e[i]), float(w[i])) for i in range(got)]


def moe_run_q8(hs, m: int, hidden: int, inter: int, n_exp: int, top_k: int, router, gate, up, down,
               shared=None, scoring: int = 0, select: int = 0, n_group: int = 1, topk_group: int = 1,
               norm_topk: bool = False, scale: float = 1.0, bias=None, L=None) -> np.ndarray:
    """Moe::run (model/ffn.rs:615-708) with every weight q8.  router, gate, up,
    down and the shared (gate, up, down) are (scales, qs) pairs; gate/up hold
    every expert's rows stacked ([n_exp*inter, hidden]), down likewise
    ([n_exp*hidden, inter]); shared is None or ((s, q), (s, q), (s, q), width)."""
    L = L or lib
    out = np.empty(m * hidden, np.float32)
    f = lambda a: _c(a, np.float32)
    i8 = lambda a: _c(a, np.int8)
    if shared is None:
        sh = [None] * 6
        sh_inter = 0
    else:
        (sgs, sgq), (sus, suq), (sds, sdq), sh_inter = shared
        sh = [f(sgs), i8(sgq), f(sus), i8(suq), f(sds), i8(sdq)]
    b = None if bias is None else f(bias)
    args = [f(router[0]), i8(router[1]), f(gate[0]), i8(gate[1]), f(up[0]), i8(up[1]), f(down[0]), i8(down[1])]
    L.kvo_moe_run_q8(P(f(hs)), m, hidden, inter, n_exp, top_k, scoring, select, n_group, topk_group,
                     int(norm_topk), scale, P(b), *[P(a) for a in args], sh_inter, *[P(a) for a in sh], P(out))
    return out


class Llm:
    """A Llama-family decoder on the CPU: the forward of
    crates/llm/src/model/llama.rs:224-289 between the embedding and the head
    (llama.rs:384-415), every operator the oracle's -- one token at a time
    (forward: run_rows with m = 1) or a prompt's pass (forward_rows:
    Transformer::forward_batch, model/mod.rs:544-549, i.e. run_rows with
    Rows::Following over m rows and the head over the last one).
    Weights are q8 (scales, qs) pairs, 1-tuples (f32 data,) -- Precision::F32,
    tensor::matvec_bt (tensor.rs:56-79) -- ("q4k", blocks) for Q4_K layer
    weights (matvec_q4k) or ("q4", scales, qs) for q4 ones (matvec_q4); norms
    and biases f32 arrays.  `L` is the oracle build its matmuls and attention
    run on (the portable one by default)."""

    def __init__(self, spec: dict, layers: list, embed, final_norm, lm_head=None, cos_t=None, sin_t=None, L=None):
        self.s, self.layers, self.embed, self.final_norm = spec, layers, embed, final_norm
        self.head = lm_head if lm_head is not None else embed
        self.cos, self.sin = cos_t, sin_t
        self.L = L
        kvd = spec["n_kv_head"] * spec["head_dim"]
        self.kc = [np.zeros((spec["n_ctx"], kvd), np.float32) for _ in layers]
        self.vc = [np.zeros((spec["n_ctx"], kvd), np.float32) for _ in layers]
        self.len = 0

    def _mm(self, w, rows, cols, xs, m, bias=None):
        """Weight::matmul_bt (quant.rs:751; m == 1 is matvec_bt, :767-769)."""
        L = self.L
        if len(w) == 1:
            return matmul_f32(w[0], rows, cols, xs, m, bias, L=L)
        if isinstance(w[0], str) and w[0] == "q4k":
            return matmul_q4k(w[1], rows, cols, xs, m, bias, L=L)
        if isinstance(w[0], str) and w[0] == "q4":
            return matmul_q4(w[1], w[2], rows, cols, xs, m, bias, L=L)
        return matmul_q8(*w, rows, cols, xs, m, bias, L=L)

    def _row(self, token: int) -> np.ndarray:
        e = self.s["n_embd"]
        if len(self.embed) == 1:                                # Weight::row, llama.rs:384-391
            return np.asarray(self.embed[0], np.float32).reshape(-1, e)[token].copy()
        return row_q8(*self.embed, e, token)

    def forward(self, token: int) -> np.ndarray:
        """One token at the next position; the logits."""
        return self.forward_rows([token])

    def forward_rows(self, tokens) -> np.ndarray:
        """A pass of m tokens at the next positions (Rows::Following): every
        projection one matmul over the m rows, each row normed, rotated and
        pushed at its own position, each row attending over the cache up to
        itself (llama.rs:249-271); the logits of the last row."""
        s = self.s
        e, hd, nh, nkv, eps = s["n_embd"], s["head_dim"], s["n_head"], s["n_kv_head"], s["eps"]
        qd, kvd, half, ff = nh * hd, nkv * hd, hd // 2, s["n_ff"]
        m, pos0 = len(tokens), self.len
        assert pos0 + m <= s["n_ctx"], "context window is full"
        xs = np.stack([self._row(int(t)) for t in tokens]).astype(np.float32)
        rope = rope_apply_interleaved if s.get("rope_interleaved") else rope_apply
        for l, Lw in enumerate(self.layers):
            hs = np.stack([rms_norm(xs[i], Lw["attn_norm"], eps) for i in range(m)])
            q = self._mm(Lw["q"], qd, e, hs, m, Lw.get("q_b")).reshape(m, qd)
            k = self._mm(Lw["k"], kvd, e, hs, m, Lw.get("k_b")).reshape(m, kvd)
            v = self._mm(Lw["v"], kvd, e, hs, m, Lw.get("v_b")).reshape(m, kvd)
            for i in range(m):                                  # llama.rs:251-257
                pos = pos0 + i
                for head in range(nh):
                    seg = q[i, head * hd:(head + 1) * hd]
                    if Lw.get("q_norm") is not None:
                        seg = rms_norm(seg, Lw["q_norm"], eps)
                    q[i, head * hd:(head + 1) * hd] = rope(self.cos, self.sin, half, seg, pos)
                for head in range(nkv):
                    seg = k[i, head * hd:(head + 1) * hd]
                    if Lw.get("k_norm") is not None:
                        seg = rms_norm(seg, Lw["k_norm"], eps)
                    k[i, head * hd:(head + 1) * hd] = rope(self.cos, self.sin, half, seg, pos)
                self.kc[l][pos], self.vc[l][pos] = k[i], v[i]   # KvCache::push
            att = np.stack([attend(nh, nkv, hd, q[i], self.kc[l][:pos0 + i + 1].ravel(),
                                   self.vc[l][:pos0 + i + 1].ravel(), pos0 + i + 1, L=self.L) for i in range(m)])
            xs = (xs + self._mm(Lw["o"], e, qd, att, m).reshape(m, e)).astype(np.float32)
            hs = np.stack([rms_norm(xs[i], Lw["mlp_norm"], eps) for i in range(m)])
            g = self._mm(Lw["gate"], ff, e, hs, m).reshape(m, ff)
            u = self._mm(Lw["up"], ff, e, hs, m).reshape(m, ff)
            xs = (xs + self._mm(Lw["down"], e, ff, swiglu(g, u), m).reshape(m, e)).astype(np.float32)
        self.len += m
        return self._mm(self.head, s["vocab"], e, rms_norm(xs[m - 1], self.final_norm, eps), 1)

    def forward_tokens(self, tokens, chunk: int = 64) -> np.ndarray:
        """Session::forward (CpuSession, model/mod.rs:1149-1158): passes of
        `chunk` tokens (KVAD_PREFILL_CHUNK's default, :1004-1006); the last
        pass's logits."""
        out = None
        for at in range(0, len(tokens), chunk):
            out = self.forward_rows(tokens[at:at + chunk])
        return out


def argmax(v) -> int:
    """sampler::argmax (crates/llm/src/sampler.rs:217-226): the first of equal
    maxima; NaN never replaces the running best."""
    v = np.asarray(v)
    if v.size == 0:
        return 0
    best, top = 0, v[0]
    for i in range(1, v.size):
        if v[i] > top:
            best, top = i, v[i]
    return best

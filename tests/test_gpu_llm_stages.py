"""Stage-by-stage parity of the decode session's layers (the forward of
crates/llm/src/model/llama.rs:224-289, embedding and head :384-415) against
the CPU oracle, through the C ABI's parity hook kh_debug_llm_trace.

test_gpu_llm.py holds the session's logits to 2e-3 x max|ref|, because an
activation requantised at the next projection can take the neighbouring int8
code.  Here each stage of every layer is held to its own bar on the device's
OWN inputs to that stage, so a wiring, norm, RoPE, cache or residual slip
cannot hide under the looser bar:

  embedding         Weight::row of the token                      exact
  q, k, v           rms_norm(x) -> GEMVs (+ biases)               1e-5
  cache push        head norms + RoPE of the device's k; its v    1e-6 / exact
  attention         device q (normed, roped) over the device's
                    cache, model::attend (mod.rs:769-819)          1e-5
  o + residual      x + o(device attention)                       1e-5
  gate, up          rms_norm(device x) -> GEMVs                   1e-5
  down + residual   x + down(quantised swiglu(device gate, up))   1e-5
  head              rms_norm(device x) -> lm_head GEMV            1e-5

GEMV references are float64 sums over the oracle's exact integer block dots,
sum_b ws[r, b] * xs[b] * dot[r, b], from the oracle's activation codes.
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

import kvad_amd as K  # noqa: E402,F401

from test_gpu_gemv import say  # noqa: E402
from test_gpu_llm import build  # noqa: E402
from test_gpu_moe_stages import close, mv  # noqa: E402


def close_residual(x_new, x_old, y, what):
    """x_new = x_old + y in f32: y held to 1e-5 x max|y|, plus the rounding of
    the f32 add (half an ulp of x_new)."""
    got = np.asarray(x_new, np.float64) - np.asarray(x_old, np.float64)
    y = np.asarray(y, np.float64)
    scale = float(np.max(np.abs(y)))
    err = float(np.max(np.abs(got - y)))
    ulp = float(np.max(np.spacing(np.abs(np.asarray(x_new, np.float32)))))
    assert err <= 1e-5 * scale + ulp / 2, f"{what}: max err {err:.3e} vs scale {scale:.3e}, ulp {ulp:.1e}"
    return max(err - ulp / 2, 0.0) / scale


def proj(w, rows, cols, x, bias=None):
    y = mv(w[0], w[1], rows, cols, x)
    return y if bias is None else y + np.asarray(bias, np.float64)


VARIANTS = {
    "qwen2": dict(bias=True),
    "qwen3": dict(bias=False, qk_norm=True, tied=False),
    "llama_interleaved": dict(bias=False, interleaved=True, n_head=8, n_kv_head=2, head_dim=128, n_embd=256),
}


def check_stages(m, ref, tokens):
    """Every stage of every layer of each token's step, on the device's own
    inputs to that stage, at the bars above; the worst relative error per
    stage."""
    s = ref.s
    e, hd, nh, nkv, eps = s["n_embd"], s["head_dim"], s["n_head"], s["n_kv_head"], s["eps"]
    qd, kvd, half, ff = nh * hd, nkv * hd, hd // 2, s["n_ff"]
    rope = O.rope_apply_interleaved if s.get("rope_interleaved") else O.rope_apply
    worst = {}
    note = lambda name, r: worst.__setitem__(name, max(worst.get(name, 0.0), r))
    for pos, tok in enumerate(tokens):
        tr = m.trace(tok)
        np.testing.assert_array_equal(tr["x_embed"], O.row_q8(*ref.embed, e, tok), err_msg="embedding")
        x = tr["x_embed"]
        for l, L in enumerate(ref.layers):
            where = f"pos {pos} layer {l}"
            h = O.rms_norm(x, L["attn_norm"], eps)
            qkv = tr["qkv"][l]
            note("q", close(qkv[:qd], proj(L["q"], qd, e, h, L.get("q_b")), f"{where} q"))
            note("k", close(qkv[qd:qd + kvd], proj(L["k"], kvd, e, h, L.get("k_b")), f"{where} k"))
            note("v", close(qkv[qd + kvd:], proj(L["v"], kvd, e, h, L.get("v_b")), f"{where} v"))
            # the push: this position's k, head-normed and roped; v as it is
            q, k = qkv[:qd].copy(), qkv[qd:qd + kvd].copy()
            for head in range(nkv):
                seg = k[head * hd:(head + 1) * hd]
                if L.get("k_norm") is not None:
                    seg = O.rms_norm(seg, L["k_norm"], eps)
                k[head * hd:(head + 1) * hd] = rope(ref.cos, ref.sin, half, seg, pos)
            for head in range(nh):
                seg = q[head * hd:(head + 1) * hd]
                if L.get("q_norm") is not None:
                    seg = O.rms_norm(seg, L["q_norm"], eps)
                q[head * hd:(head + 1) * hd] = rope(ref.cos, ref.sin, half, seg, pos)
            kc, vc = tr["k_cache"][l], tr["v_cache"][l]
            note("k push", close(kc[pos], k, f"{where} k push", rtol=1e-6))
            np.testing.assert_array_equal(vc[pos], qkv[qd + kvd:], err_msg=f"{where} v push")
            att = O.attend(nh, nkv, hd, q, kc.ravel(), vc.ravel(), pos + 1)
            note("attention", close(tr["att"][l], att, f"{where} attention"))
            y = proj(L["o"], e, qd, tr["att"][l])
            note("o + x", close_residual(tr["x_attn"][l], x, y, f"{where} o + residual"))
            x = tr["x_attn"][l]
            h = O.rms_norm(x, L["mlp_norm"], eps)
            note("gate", close(tr["gate"][l], proj(L["gate"], ff, e, h), f"{where} gate"))
            note("up", close(tr["up"][l], proj(L["up"], ff, e, h), f"{where} up"))
            y = proj(L["down"], e, ff, O.swiglu(tr["gate"][l], tr["up"][l]))
            note("down + x", close_residual(tr["x_mlp"][l], x, y, f"{where} down + residual"))
            x = tr["x_mlp"][l]
        logits = proj(ref.head, s["vocab"], e, O.rms_norm(x, ref.final_norm, eps))
        note("head", close(tr["logits"], logits, f"pos {pos} head"))
    return worst


@pytest.mark.parametrize("variant", list(VARIANTS))
def test_each_stage_of_every_layer(ctx, variant):
    say("llm stages", variant)
    m, mk = build(ctx, 170, n_layer=3, **VARIANTS[variant])
    worst = check_stages(m, mk(), [3, 17, 500, 42, 7, 7, 99])
    say("llm stages worst", variant, {k: f"{v:.1e}" for k, v in worst.items()})


def test_each_stage_at_qwen05b_width_and_depth(ctx):
    # Qwen2.5-0.5B's widths and depth (24 layers, 896 / 14 / 2 x 64 / 4864,
    # q/k/v biases; a 4096-token vocabulary): every stage of every layer
    # holds its bar at the size the benchmark runs, where the logits against
    # the oracle's own chain drift further than at two layers (each
    # requantised activation can take the neighbouring code; 24 layers of
    # them compound): that drift is the chain's, not any stage's.
    say("llm stages at Qwen2.5-0.5B width")
    m, mk = build(ctx, 180, n_layer=24, n_embd=896, n_head=14, n_kv_head=2, head_dim=64, n_ff=4864, vocab=4096,
                  n_ctx=64)
    ref = mk()
    worst = check_stages(m, ref, [3, 17, 500])
    say("llm stages worst (Qwen width)", {k: f"{v:.1e}" for k, v in worst.items()})

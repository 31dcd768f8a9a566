"""A prompt read on the device a pass at a time: Session::forward(&[u32])
(crates/llm/src/model/mod.rs:842; CpuSession :1149-1158) over
forward_batch (mod.rs:544-549) = embedding rows, run_rows with
Rows::Following (llama.rs:224-289) and the head over the last row
(llama.rs:404-411); Session::prefill_pass (mod.rs:866, :1181-1183) and
CpuSession::reading (mod.rs:1079-1082); through the C ABI.

The reference's own case (crates/llm/tests/batched_decode.rs:261-290): a
23-token prompt read five tokens a pass, with the passes cut where
prefill_pass says, gives the logits of the prompt read in one call to the
bit, the same cache length, and the same next-token logits.  Beyond it:

  * logits after the prompt against the oracle's forward, token at a time
    (the reference's x86 matmul is row-by-row qrow, so a pass and m single
    steps are the same arithmetic there), at the session bar 2e-3 x max, with
    the next token the argmax of those logits exactly; passes on the
    multi-token GEMV (<= 32 rows) and on the int8 / f32 GEMM (> 32 rows);
    the attention on the pass kernel (every row's whole sequence in one
    workgroup, the default; its positions dealt over 1, 2, 4 or 8 waves,
    KVAD_PASS_WAVES) and, with KVAD_PASS_ATTN=0, on the rows launch as
    one split and as split + merged; a prompt past the single-split line
    (300 positions) both ways;
  * every stage of every layer of a pass on the device's own inputs, through
    kh_debug_llm_trace_pass, at the stage bars of test_gpu_llm_stages
    (projections 1e-5, the pushed keys 1e-6 and values exact, attention of
    row i over len + i + 1 positions 1e-5, residuals 1e-5 + half an ulp);
  * decode after a prompt: the captured steps continue from the pass's state;
  * refusals: tokens out of range and prompts past n_ctx leave the session
    as it was; an empty prompt does nothing.
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

import kvad_amd as K  # noqa: E402

from test_gpu_gemv import say  # noqa: E402
from test_gpu_llm import LOGIT_RTOL, build  # noqa: E402
from test_gpu_llm_stages import close_residual, proj  # noqa: E402
from test_gpu_moe_stages import close  # noqa: E402

VARIANTS = {
    # batched_decode.rs:264: ("llama", F32), ("qwen3", Q8)
    "llama_f32": dict(bias=False, interleaved=True, tied=False, prec="f32"),
    "qwen3_q8": dict(bias=False, qk_norm=True, tied=False),
    "qwen2_q8": dict(bias=True),
    "llama_hd128_q8": dict(bias=False, interleaved=True, n_head=8, n_kv_head=2, head_dim=128, n_embd=256),
    "llama_q4k": dict(bias=False, interleaved=True, n_head=4, n_kv_head=2, head_dim=64, n_embd=256, n_ff=512,
                      prec="q4k"),
    "qwen2_q4": dict(bias=True, prec="q4"),
    # head layouts the pass kernel tiles differently (16 columns = rows x
    # the group's query heads): MHA (16 rows a tile), Qwen2.5-0.5B's group
    # of 7 (2 rows, 14 columns), MQA with 16 heads (1 row)
    "mha_q8": dict(bias=False, n_head=4, n_kv_head=4),
    "gqa7_q8": dict(bias=True, n_head=14, n_kv_head=2, n_embd=256),
    "mqa16_q8": dict(bias=False, n_head=16, n_kv_head=1, n_embd=256),
}

PROMPT = [(i * 7 + 3) % 512 for i in range(23)]  # batched_decode.rs:263 (VOCAB = 512 here)


def logits_close(got, want, what):
    scale = float(np.max(np.abs(want)))
    err = float(np.max(np.abs(np.asarray(got, np.float64) - want)))
    assert np.all(np.isfinite(got)), f"{what}: not finite"
    assert err <= LOGIT_RTOL * scale, f"{what}: max err {err:.3e} vs scale {scale:.3e}"
    return err / scale


@pytest.mark.parametrize("variant", list(VARIANTS))
def test_a_prompt_read_a_pass_at_a_time_is_the_prompt_read_at_once(ctx, variant):
    say("prefill passes vs once", variant)
    once, _ = build(ctx, 300, **VARIANTS[variant])
    passes, _ = build(ctx, 300, **VARIANTS[variant])
    once.reading(5)  # five tokens a pass: four whole passes and three left over
    passes.reading(5)
    want, want_next = once.forward_tokens(PROMPT)
    at, count, got, got_next = 0, 0, None, None
    while at < len(PROMPT):
        n = passes.prefill_pass(len(PROMPT) - at)
        assert 1 <= n <= len(PROMPT) - at, f"a pass of {n} with {len(PROMPT) - at} left"
        got, got_next = passes.forward_tokens(PROMPT[at:at + n])
        at += n
        count += 1
    assert count == 5, f"{variant}: the prompt was not read in passes"
    assert len(passes) == len(once) == len(PROMPT)
    np.testing.assert_array_equal(got, want, err_msg=f"{variant}: a pass at a time changed the logits")
    assert got_next == want_next
    # and the next token after it agrees too, so the caches do
    a, na = passes.forward_tokens([9])
    b, nb = once.forward_tokens([9])
    np.testing.assert_array_equal(a, b)
    assert na == nb


def test_prefill_pass_cuts_whole_chunks_from_the_front(ctx, monkeypatch):
    say("prefill_pass")
    m, _ = build(ctx, 301)
    # the default: 512 a pass, the reference's GPU backend's chunk (gpu/src/model.rs:897)
    assert [m.prefill_pass(n) for n in (1, 63, 512, 513, 2000)] == [1, 63, 512, 512, 512]
    m.reading(5)
    assert [m.prefill_pass(n) for n in (23, 5, 3, 0)] == [5, 5, 3, 0]
    m.reading(0)
    monkeypatch.setenv("KVAD_PREFILL_CHUNK", "16")
    assert m.prefill_pass(40) == 16
    with pytest.raises(K.KvadError):
        m.reading(1 << 16)


CASES = {
    # (variant, prompt length, chunk, attention: the pass kernel, or the
    # rows launch as one split or split + merged)
    "gemv_rows": ("qwen2_q8", 23, 64, "pass"),       # one pass of 23 rows: multi-token GEMVs
    "gemv_rows_single": ("qwen2_q8", 23, 64, "single"),
    "gemm_rows": ("qwen2_q8", 40, 40, "single"),     # one pass of 40 rows: the int8 GEMM
    "gemm_pass": ("qwen3_q8", 40, 40, "pass"),
    "gemm_split": ("qwen3_q8", 40, 40, "split"),     # every row split and merged
    "f32_gemm": ("llama_f32", 40, 40, "pass"),       # the f32 GEMM
    "q4k_gemm": ("llama_q4k", 37, 64, "pass"),
    "q4_passes": ("qwen2_q4", 23, 7, "pass"),
    "hd128_passes": ("llama_hd128_q8", 30, 8, "pass"),
    "hd128_passes_w8": ("llama_hd128_q8", 30, 8, "pass:8"),
    "hd128_split": ("llama_hd128_q8", 30, 8, "split"),
    "gemm_pass_w4": ("qwen2_q8", 40, 40, "pass:4"),
}


def attention_path(monkeypatch, attn):
    # "pass" (waves per workgroup by the launch's rule), "pass:W" (W waves),
    # "single" / "split": the rows launch
    if attn.startswith("pass:"):
        monkeypatch.setenv("KVAD_PASS_WAVES", attn[5:])
    elif attn != "pass":
        monkeypatch.setenv("KVAD_PASS_ATTN", "0")
    if attn == "split":
        monkeypatch.setenv("KVAD_ATTN_SINGLE", "0")


@pytest.mark.parametrize("case", list(CASES))
def test_prefill_matches_the_oracle(ctx, monkeypatch, case):
    variant, n, chunk, attn = CASES[case]
    attention_path(monkeypatch, attn)
    say("prefill vs oracle", case)
    m, mk = build(ctx, 310, **VARIANTS[variant])
    m.reading(chunk)
    ref = mk()
    prompt = [(i * 13 + 5) % 512 for i in range(n)]
    logits, nxt = m.forward_tokens(prompt)
    for t in prompt:
        want = ref.forward(t)
    worst = logits_close(logits, want, f"{case} after the prompt")
    assert nxt == O.argmax(logits), "the next token is not the argmax of the last logits"
    assert len(m) == n
    # decoding goes on from the prompt's cache
    for step, t in enumerate([nxt, 9, 400]):
        lg, nt = m.forward(int(t))
        worst = max(worst, logits_close(lg, ref.forward(int(t)), f"{case} decode step {step}"))
        assert nt == O.argmax(lg)
    say("prefill vs oracle worst", case, f"{worst:.2e}")


@pytest.mark.parametrize("attn", ["pass", "pass:8", "single"])
@pytest.mark.parametrize("chunk", [64, 512])
def test_a_prompt_past_the_single_split_line(ctx, monkeypatch, chunk, attn):
    # 300 positions at head_dim 64: passes of 64 rows, or one pass of 300
    # rows, on the pass kernel or on the rows launch (one split up to 256
    # positions, split + merged past them)
    attention_path(monkeypatch, attn)
    say("prefill past the single split", chunk, attn)
    m, mk = build(ctx, 320, n_layer=1, n_ctx=512)
    m.reading(chunk)
    ref = mk()
    prompt = [(i * 11 + 2) % 512 for i in range(300)]
    logits, nxt = m.forward_tokens(prompt)
    for t in prompt:
        want = ref.forward(t)
    logits_close(logits, want, "after 300 tokens")
    assert nxt == O.argmax(logits) and len(m) == 300


def test_generation_continues_from_the_prompt(ctx):
    say("prefill then generate")
    a, _ = build(ctx, 330)
    b, _ = build(ctx, 330)
    _, na = a.forward_tokens(PROMPT)
    _, nb = b.forward_tokens(PROMPT)
    assert na == nb
    got = a.generate(na, 8)  # the captured step from the pass's state
    t, want = nb, []
    for _ in range(8):
        _, t = b.forward(t)
        want.append(t)
    np.testing.assert_array_equal(got, want)


def test_refusals_leave_the_session_as_it_was(ctx):
    say("prefill refusals")
    m, _ = build(ctx, 340, n_ctx=32)
    plain, _ = build(ctx, 340, n_ctx=32)
    m.forward_tokens([1, 2, 3])
    plain.forward_tokens([1, 2, 3])
    with pytest.raises(K.KvadError, match="out of range"):
        m.forward_tokens([4, 512, 6])
    with pytest.raises(K.KvadError, match="overrun"):
        m.forward_tokens(list(range(30)))
    lg, nt = m.forward_tokens([])
    assert len(m) == 3
    a, na = m.forward_tokens([7, 8])
    b, nb = plain.forward_tokens([7, 8])
    np.testing.assert_array_equal(a, b)
    assert na == nb


STAGE_VARIANTS = {
    # (variant, positions held, rows in the pass, attention)
    "qwen2_gemv": ("qwen2_q8", 3, 6, "pass"),          # 3 positions held, a pass of 6 rows
    "qwen3_gemm": ("qwen3_q8", 2, 40, "pass"),         # a pass of 40 rows on the int8 GEMM
    "qwen3_gemm_rows": ("qwen3_q8", 2, 40, "single"),
    "llama_hd128": ("llama_hd128_q8", 4, 12, "pass"),
    "llama_hd128_split": ("llama_hd128_q8", 4, 12, "split"),
    "qwen2_long": ("qwen2_q8", 70, 37, "pass"),        # rows over 71 .. 107 positions
    "qwen2_long_w2": ("qwen2_q8", 70, 37, "pass:2"),   # the positions dealt over 2, 4, 8 waves
    "qwen2_long_w4": ("qwen2_q8", 70, 37, "pass:4"),
    "qwen2_long_w8": ("qwen2_q8", 70, 37, "pass:8"),
    "hd128_long_w4": ("llama_hd128_q8", 50, 21, "pass:4"),
    "mha": ("mha_q8", 5, 37, "pass"),
    "gqa7": ("gqa7_q8", 5, 37, "pass:4"),
    "mqa16": ("mqa16_q8", 5, 37, "pass:2"),
}


@pytest.mark.parametrize("case", list(STAGE_VARIANTS))
def test_each_stage_of_a_pass(ctx, monkeypatch, case):
    variant, held, n, attn = STAGE_VARIANTS[case]
    attention_path(monkeypatch, attn)
    say("prefill stages", case)
    m, mk = build(ctx, 350, n_layer=3, n_ctx=max(64, held + n), **VARIANTS[variant])
    ref = mk()  # for its weights, norms and tables only
    s = ref.s
    e, hd, nh, nkv, eps = s["n_embd"], s["head_dim"], s["n_head"], s["n_kv_head"], s["eps"]
    qd, kvd, half, ff = nh * hd, nkv * hd, hd // 2, s["n_ff"]
    rope = O.rope_apply_interleaved if s.get("rope_interleaved") else O.rope_apply
    if held:
        m.forward_tokens([(i * 5 + 1) % 512 for i in range(held)])
    toks = [(i * 17 + 4) % 512 for i in range(n)]
    tr = m.trace_pass(toks)
    assert len(m) == held + n
    worst = {}
    note = lambda name, r: worst.__setitem__(name, max(worst.get(name, 0.0), r))
    for i, t in enumerate(toks):
        np.testing.assert_array_equal(tr["x_embed"][i], O.row_q8(*ref.embed, e, t), err_msg=f"embedding row {i}")
    X = tr["x_embed"]
    for l, L in enumerate(ref.layers):
        X_attn, X_mlp = tr["x_attn"][l], tr["x_mlp"][l]
        kc, vc = tr["k_cache"][l], tr["v_cache"][l]
        for i in range(n):
            pos, where = held + i, f"layer {l} row {i}"
            x = X[i]
            h = O.rms_norm(x, L["attn_norm"], eps)
            qkv = tr["qkv"][l][i]
            note("q", close(qkv[:qd], proj(L["q"], qd, e, h, L.get("q_b")), f"{where} q"))
            note("k", close(qkv[qd:qd + kvd], proj(L["k"], kvd, e, h, L.get("k_b")), f"{where} k"))
            note("v", close(qkv[qd + kvd:], proj(L["v"], kvd, e, h, L.get("v_b")), f"{where} v"))
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
            note("k push", close(kc[pos], k, f"{where} k push", rtol=1e-6))
            np.testing.assert_array_equal(vc[pos], qkv[qd + kvd:], err_msg=f"{where} v push")
            # row i attends over the held positions and the pass's rows up to itself
            att = O.attend(nh, nkv, hd, q, kc[:pos + 1].ravel(), vc[:pos + 1].ravel(), pos + 1)
            note("attention", close(tr["att"][l][i], att, f"{where} attention"))
            y = proj(L["o"], e, qd, tr["att"][l][i])
            note("o + x", close_residual(X_attn[i], x, y, f"{where} o + residual"))
            h = O.rms_norm(X_attn[i], L["mlp_norm"], eps)
            note("gate", close(tr["gate"][l][i], proj(L["gate"], ff, e, h), f"{where} gate"))
            note("up", close(tr["up"][l][i], proj(L["up"], ff, e, h), f"{where} up"))
            y = proj(L["down"], e, ff, O.swiglu(tr["gate"][l][i], tr["up"][l][i]))
            note("down + x", close_residual(X_mlp[i], X_attn[i], y, f"{where} down + residual"))
        X = X_mlp
    logits = proj(ref.head, s["vocab"], e, O.rms_norm(X[n - 1], ref.final_norm, eps))
    note("head", close(tr["logits"], logits, "head of the last row"))
    say("prefill stages worst", case, {k: f"{v:.1e}" for k, v in worst.items()})

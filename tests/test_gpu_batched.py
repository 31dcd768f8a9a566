"""Batched decode on the device: several conversations advanced by one token
in one pass (Session::forward_each, crates/llm/src/model/mod.rs:899-930 and
:1190-1202; Transformer::forward_each, llama.rs:418-434), with the sessions'
park / resume (mod.rs:883-897, :1204-1212), through the C ABI.

The cases follow the reference's own (crates/llm/tests/batched_decode.rs):
conversations of DIFFERENT lengths, so that a row reading another
conversation's history, or its own at the wrong position, cannot pass; each
row's logits held to the same conversation stepped alone (resume, one token,
park) -- the reference's criterion, :141-176 and :202-240 -- and to the
oracle's forward of that conversation (q8 and f32 weights).  A batch of one is a
token and a batch of none is nothing (:190-200); the session's own
conversation is untouched by the batched step (:209-215).

Bar.  Rows against the same conversation alone: 2e-3 x max|logit|, the
reference's `close` bar (:134-139; the batched pass quantises each row
exactly as the single step does, but sums in another order).  Against the
oracle: 2e-3 x max, as in test_gpu_llm.  The next token is the argmax of the
row's own logits, exactly.
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

import kvad_amd as K  # noqa: E402

from test_gpu_gemv import say  # noqa: E402
from test_gpu_llm import LOGIT_RTOL, build  # noqa: E402

PROMPTS = [[3, 17, 8, 0, 29, 41, 5], [12], [60, 2, 2, 33]]  # batched_decode.rs:141
NEXT = [[7, 7, 7], [1, 44, 19], [63, 0, 30], [9, 21, 9]]    # batched_decode.rs:142


def close(got, want, what):
    scale = float(np.max(np.abs(want)))
    err = float(np.max(np.abs(np.asarray(got, np.float64) - want)))
    assert np.all(np.isfinite(got)), f"{what}: not finite"
    assert err <= LOGIT_RTOL * scale, f"{what}: max err {err:.3e} vs scale {scale:.3e}"


def set_aside(m, prompts):
    """Each prompt fed one token at a time, then parked; the session then
    holds a conversation of its own, [5, 6] (batched_decode.rs:209-222)."""
    parked = []
    for p in prompts:
        for t in p:
            m.forward(t, want_logits=False)
        parked.append(m.park())
    for t in (5, 6):
        m.forward(t, want_logits=False)
    return parked


VARIANTS = {
    "qwen2_q8": dict(bias=True),
    "qwen3_q8": dict(bias=False, qk_norm=True, tied=False),
    "llama_hd128_q8": dict(bias=False, interleaved=True, n_head=8, n_kv_head=2, head_dim=128, n_embd=256),
    "qwen2_f32": dict(bias=True, tied=False, prec="f32"),  # every projection on the f32 GEMM / GEMV
    # Q4_K and q4 layer weights (embedding and head q8), 256-multiple widths
    "llama_q4k": dict(bias=False, interleaved=True, n_head=4, n_kv_head=2, head_dim=64, n_embd=256, n_ff=512,
                      prec="q4k"),
    "qwen2_q4": dict(bias=True, prec="q4"),
}


@pytest.mark.parametrize("attn", ["single", "split"])
@pytest.mark.parametrize("variant", list(VARIANTS))
def test_several_conversations_at_once_say_what_each_says_alone(ctx, monkeypatch, variant, attn):
    # every row's attention as one split, or (KVAD_ATTN_SINGLE=0) split and merged
    if attn == "split":
        monkeypatch.setenv("KVAD_ATTN_SINGLE", "0")
    say("forward_each vs alone", variant, attn)
    one, mk = build(ctx, 700, **VARIANTS[variant])
    alle, _ = build(ctx, 700, **VARIANTS[variant])
    theirs, ours = set_aside(one, PROMPTS), set_aside(alle, PROMPTS)
    refs = [mk() for _ in PROMPTS]
    for r, p in zip(refs, PROMPTS):
        for t in p:
            r.forward(t)
    for step, tokens in enumerate(NEXT):
        got, nxt = alle.forward_each(tokens, ours)
        assert got.shape == (len(tokens), alle.spec.vocab)
        assert len(alle) == 2, "the session's own conversation moved"
        own = one.park()
        for i, t in enumerate(tokens):
            one.resume(theirs[i])
            want, _ = one.forward(t)
            theirs[i] = one.park()
            close(got[i], want, f"{variant} step {step} conversation {i} vs alone")
            assert len(ours[i]) == len(theirs[i]) == len(PROMPTS[i]) + step + 1
            assert nxt[i] == O.argmax(got[i]), f"step {step} row {i}: next is not the row's argmax"
            close(got[i], refs[i].forward(t), f"{variant} step {step} conversation {i} vs oracle")
        one.resume(own)


def test_the_sessions_own_conversation_is_left_as_it_was(ctx):
    say("forward_each leaves the held conversation")
    m, _ = build(ctx, 710)
    plain, _ = build(ctx, 710)
    parked = set_aside(m, PROMPTS)
    for t in (5, 6):
        plain.forward(t, want_logits=False)
    for tokens in NEXT:
        m.forward_each(tokens, parked, want_logits=False)
    a, na = m.forward(9)
    b, nb = plain.forward(9)
    np.testing.assert_array_equal(a, b)
    assert na == nb and len(m) == len(plain) == 3


def test_park_and_resume_continue_bit_for_bit(ctx):
    say("park / resume")
    m, _ = build(ctx, 720)
    plain, _ = build(ctx, 720)
    for t in (4, 8, 15):
        m.forward(t, want_logits=False)
        plain.forward(t, want_logits=False)
    p = m.park()
    assert len(m) == 0 and len(p) == 3
    for t in (16, 23):  # another conversation meanwhile
        m.forward(t, want_logits=False)
    m.resume(p)
    assert len(m) == 3
    for t in (42, 1):
        np.testing.assert_array_equal(m.forward(t)[0], plain.forward(t)[0])
    # generate (a captured graph) after a park/resume names the held cache
    np.testing.assert_array_equal(m.generate(3, 4), plain.generate(3, 4))


def test_a_batch_of_one_is_a_token_and_a_batch_of_none_is_nothing(ctx):
    say("forward_each of one and of none")
    m, _ = build(ctx, 730)
    a = set_aside(m, [PROMPTS[0]])
    plain, _ = build(ctx, 730)
    for t in PROMPTS[0]:
        plain.forward(t, want_logits=False)
    got, nxt = m.forward_each([11], a)
    want, wn = plain.forward(11)
    close(got[0], want, "one")
    assert nxt[0] == O.argmax(got[0])
    got, nxt = m.forward_each([], [])
    assert got.shape == (0, m.spec.vocab) and nxt.size == 0


ROW_CASES = {
    "q8_8": (8, {}), "q8_13": (13, {}), "q8_20": (20, {}), "q8_40": (40, {}),
    # the down projection's 1024-wide input is eight k-stages: at 40 rows the
    # GEMM splits them over the grid and the last split adds the residual
    "q8_40_split": (40, dict(n_ff=1024)),
    "q4k_5": (5, dict(prec="q4k", n_embd=256, n_ff=512)), "q4k_20": (20, dict(prec="q4k", n_embd=256, n_ff=512)),
    "q4k_40": (40, dict(prec="q4k", n_embd=256, n_ff=1024)),
    "q4_6": (6, dict(prec="q4")), "q4_40": (40, dict(prec="q4", n_ff=1024)),
}


@pytest.mark.parametrize("case", list(ROW_CASES))
def test_many_rows_on_the_multi_token_gemv_and_the_gemm(ctx, case):
    # up to 16 rows: one multi-token GEMV launch per projection group (on
    # the matrix cores from five rows); 20: two launches; 40: the int8 GEMM,
    # residual added in its epilogue (q8, q4 and Q4_K layer weights)
    n, kw = ROW_CASES[case]
    say("forward_each rows", case)
    m, mk = build(ctx, 740 + n, **kw)
    prompts = [[(7 * i + j) % 500 for j in range(1 + (5 * i) % 11)] for i in range(n)]
    parked = set_aside(m, prompts)
    refs = [mk() for _ in prompts]
    for r, p in zip(refs, prompts):
        for t in p:
            r.forward(t)
    for step in range(2):
        tokens = [(31 * i + 3 * step) % 512 for i in range(n)]
        got, nxt = m.forward_each(tokens, parked)
        for i, t in enumerate(tokens):
            close(got[i], refs[i].forward(t), f"rows {n} step {step} conversation {i}")
            assert nxt[i] == O.argmax(got[i])


@pytest.mark.parametrize("attn", ["single", "split"])
def test_long_conversations_attend_across_many_splits(ctx, monkeypatch, attn):
    # lengths 1..300 in one pass: rows of one split and rows of several; or
    # lengths 1..251, every row's attention one split (the pass is bucketed
    # by its longest row)
    monkeypatch.delenv("KVAD_ATTN_SINGLE", raising=False)
    say("forward_each long", attn)
    m, mk = build(ctx, 760, n_ctx=512)
    lens = [300, 1, 129, 64, 65] if attn == "split" else [250, 1, 129, 64, 65]
    prompts = [[(13 * i + 5 * j) % 512 for j in range(L)] for i, L in enumerate(lens)]
    parked = set_aside(m, prompts)
    refs = [mk() for _ in prompts]
    for r, p in zip(refs, prompts):
        for t in p:
            r.forward(t)
    tokens = [2, 4, 6, 8, 10]
    got, _ = m.forward_each(tokens, parked)
    for i, t in enumerate(tokens):
        close(got[i], refs[i].forward(t), f"long conversation {i} (length {lens[i]})")


def test_refusals(ctx):
    say("forward_each refusals")
    m, _ = build(ctx, 780, n_ctx=4)
    other, _ = build(ctx, 781)
    a, b = set_aside(m, [[1], [2]])[:2]
    x = other.park()
    with pytest.raises(K.KvadError, match="twice"):
        m.forward_each([1, 2], [a, a])
    with pytest.raises(K.KvadError, match="not this backend"):
        m.forward_each([1, 2], [a, x])
    with pytest.raises(K.KvadError, match="out of range"):
        m.forward_each([1, 9999], [a, b])
    with pytest.raises(K.KvadError, match="a token for each"):
        m.forward_each([1], [a, b])
    for _ in range(3):
        m.forward_each([1, 2], [a, b], want_logits=False)
    assert len(a) == 4
    with pytest.raises(K.KvadError, match="full"):
        m.forward_each([1, 2], [a, b])
    with pytest.raises(K.KvadError, match="not this backend"):
        m.resume(x)  # consumed even though refused
    assert x.h is None

"""The greedy choice at the end of the device step (sampler::argmax,
crates/llm/src/sampler.rs:217-226: the first of equal maxima; a NaN never
replaces the running best, and a NaN first entry keeps index 0) on planted
heads, through the C ABI.

The head GEMV's workgroups each keep their best row; the last to finish
takes the best of them and row 0 (KVAD_HEAD_TAIL=1, the default), or a
one-workgroup launch after the GEMV does (KVAD_HEAD_TAIL=0).  Random logits
never exercise the rules that matter there, so the head is planted: the
step's largest row copied into rows in other workgroups (equal maxima across
workgroups: the lowest index wins), into row 0 (a tie with row 0: 0 wins),
into row 0 with twice its scales (row 0 the maximum), and NaN scales on the
largest row or on row 0 (NaN logits).  The first step's hidden state does not
depend on the head, so a run with the unplanted head names the largest row.
Each case checks the per-token call's next token against the oracle's
argmax of the same logits, bit-equal copies where a tie was planted, and the
captured steps (kh_llm_generate) against the per-token chain.
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

import kvad_amd as K  # noqa: E402,F401

from test_gpu_gemv import say  # noqa: E402
from test_gpu_llm import build  # noqa: E402

VOCAB = 8192
N_EMBD = 128
SEED = 910
TOKEN = 5


def plant(case, top):
    far = [3, VOCAB - 5]  # rows of other workgroups than the largest one's

    def edit(s, q):
        s = s.reshape(VOCAB, -1)
        q = q.reshape(VOCAB, N_EMBD)
        if case == "tie_across_groups":
            for r in far:
                s[r], q[r] = s[top], q[top]
        elif case == "row0_tie":
            s[0], q[0] = s[top], q[top]
        elif case == "row0_max":
            s[0], q[0] = 2.0 * s[top], q[top]
        elif case == "nan_row":
            s[top] = np.nan
        elif case == "nan_row0":
            s[0] = np.nan
        return s.reshape(-1), q.reshape(-1)

    return edit, far


CASES = ["tie_across_groups", "row0_tie", "row0_max", "nan_row", "nan_row0"]


@pytest.mark.parametrize("tail", ["1", "0"])
@pytest.mark.parametrize("case", CASES)
def test_greedy_choice_on_planted_heads(ctx, monkeypatch, case, tail):
    monkeypatch.setenv("KVAD_HEAD_TAIL", tail)
    say("greedy tail", case, "KVAD_HEAD_TAIL=" + tail)
    plain, _ = build(ctx, SEED, tied=False, vocab=VOCAB, n_embd=N_EMBD)
    base, _ = plain.forward(TOKEN)
    top = int(O.argmax(base))
    assert top not in (0, 3, VOCAB - 5), "the plant needs the largest row elsewhere"
    edit, far = plant(case, top)

    m, _ = build(ctx, SEED, tied=False, vocab=VOCAB, n_embd=N_EMBD, head_edit=edit)
    logits, nxt = m.forward(TOKEN)
    want = O.argmax(logits)
    assert nxt == want, f"{case}: the device chose {nxt}, the reference's argmax is {want}"
    if case == "tie_across_groups":
        assert all(logits[r] == logits[top] for r in far), "the planted rows do not tie"
        assert want == min(far + [top])
    elif case == "row0_tie":
        assert logits[0] == logits[top] and want == 0
    elif case == "row0_max":
        assert logits[0] > logits[top] and want == 0
    elif case == "nan_row":
        assert np.isnan(logits[top]) and want != top
    elif case == "nan_row0":
        assert np.isnan(logits[0]) and want == 0

    # the captured steps against the per-token chain
    chain, _ = build(ctx, SEED, tied=False, vocab=VOCAB, n_embd=N_EMBD, head_edit=edit)
    g, _ = build(ctx, SEED, tied=False, vocab=VOCAB, n_embd=N_EMBD, head_edit=edit)
    t, expect = TOKEN, []
    for _ in range(4):
        lg, t = chain.forward(t)
        assert t == O.argmax(lg)
        expect.append(t)
    got = g.generate(TOKEN, 4)
    np.testing.assert_array_equal(got, expect)

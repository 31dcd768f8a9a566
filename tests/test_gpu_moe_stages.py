"""Stage-by-stage parity of the mixture-of-experts layer (Moe::run,
model/ffn.rs:615-708; decode_together ffn.rs:820-842; mix ffn.rs:775-805)
against the CPU oracle, through the C ABI's parity hook kh_debug_moe_picks.

The layer's output is held to 2e-3 x max|ref| in test_gpu_moe.py because the
SwiGLU hidden is quantised again before the down projections.  Here every
arithmetic stage is held to 1e-5 x max|ref| on the device's OWN inputs to that
stage, so a mixing-order, scale or routing slip cannot hide under the looser
bar:

  router logits     x -> router GEMV                          1e-5
  routes            the device's logits -> Router::route      exact
  gate, up          x -> each picked expert's GEMV            1e-5
  shared gate, up   x -> the shared expert's GEMVs            1e-5
  hidden codes      swiglu(device gate, device up) quantised  exact but for
                    (batched path, where the codes are kept)  boundary flips,
                                                              counted
  expert out        device hidden codes -> down GEMV          1e-5
  shared out        swiglu(device shared gate, up) -> down    1e-5
  mix               shared out + sum w * expert out, in
                    expert order, from the device's stages    exact

The references of the GEMV stages are float64 sums over the oracle's integer
block dots (block_dots_q8), sum_b ws[r, b] * xs[b] * dot[r, b], from codes the
oracle's quantiser makes (bit-exact with the device's, test_gpu_golden.py).
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

import kvad_amd as K  # noqa: E402

from test_gpu_gemv import say  # noqa: E402

STAGE_RTOL = 1e-5


def close(got, want, what, rtol=STAGE_RTOL):
    want = np.asarray(want, np.float64)
    scale = max(float(np.max(np.abs(want))), 1e-30)
    err = float(np.max(np.abs(np.asarray(got, np.float64) - want)))
    assert err <= rtol * scale, f"{what}: max err {err:.3e} vs scale {scale:.3e} (rel {err / scale:.2e})"
    return err / scale


def mv_codes(s, q, rows, cols, xq, xs):
    """y = x W^T from the activation's codes: float64 over exact block dots."""
    dots = O.block_dots_q8(q, rows, cols, xq).astype(np.float64)
    ws = np.asarray(s, np.float64).reshape(rows, cols // 32)
    return (ws * dots * np.asarray(xs, np.float64)[None, :]).sum(axis=1)


def mv(s, q, rows, cols, x):
    xq, xs, _ = O.qact(x)
    return mv_codes(s, q, rows, cols, xq, xs)


class Layer:
    """A q8 MoE layer with its weights kept on the host for the references."""

    def __init__(self, ctx, hidden, inter, n_exp, top_k, seed, sh_inter=0):
        q = lambda s, r, c, sc: O.quantize_q8(O.normal(s, r * c, sc), r, c)
        self.hidden, self.inter, self.n_exp, self.top_k, self.sh = hidden, inter, n_exp, top_k, sh_inter
        self.router = q(seed, n_exp, hidden, 0.5)
        g, u, d = q(seed + 1, n_exp * inter, hidden, 0.02), q(seed + 2, n_exp * inter, hidden, 0.02), \
            q(seed + 3, n_exp * hidden, inter, 0.02)
        per = lambda a: (a[0].reshape(n_exp, -1), a[1].reshape(n_exp, -1))
        self.gate, self.up, self.down = per(g), per(u), per(d)
        self.moe = K.Moe(ctx, n_exp, top_k, hidden, inter)
        self.moe.set_router(K.Weight.from_q8(ctx, n_exp, hidden, *self.router))
        for x in range(n_exp):
            self.moe.set_expert(x, K.Weight.from_q8(ctx, inter, hidden, self.gate[0][x], self.gate[1][x]),
                                K.Weight.from_q8(ctx, inter, hidden, self.up[0][x], self.up[1][x]),
                                K.Weight.from_q8(ctx, hidden, inter, self.down[0][x], self.down[1][x]))
        if sh_inter:
            self.sg, self.su = q(seed + 4, sh_inter, hidden, 0.02), q(seed + 5, sh_inter, hidden, 0.02)
            self.sd = q(seed + 6, hidden, sh_inter, 0.02)
            self.moe.set_shared(K.Weight.from_q8(ctx, sh_inter, hidden, *self.sg),
                                K.Weight.from_q8(ctx, sh_inter, hidden, *self.su),
                                K.Weight.from_q8(ctx, hidden, sh_inter, *self.sd))


def check_stages(L, hs, m, tokens):
    """Run the layer on m tokens and hold each stage of `tokens` to its bar."""
    h, inter, k = L.hidden, L.inter, L.top_k
    out = L.moe.run(hs, m).reshape(m, h)
    st = L.moe.picks(m, hidden_codes=m > 1)
    worst, flips, codes = {}, 0, 0
    note = lambda name, r: worst.__setitem__(name, max(worst.get(name, 0.0), r))
    for t in tokens:
        x = hs[t * h:(t + 1) * h]
        note("router", close(st["logits"][t], mv(*L.router, L.n_exp, h, x), f"token {t} router logits"))
        picks = sorted(O.route(st["logits"][t], top_k=k))  # the routes, into expert order
        n = int(st["count"][t])
        assert n == len(picks)
        assert [e for e, _ in picks] == list(st["experts"][t, :n]), f"token {t}: experts"
        np.testing.assert_allclose(st["weights"][t, :n], [w for _, w in picks], rtol=1e-6, atol=0)
        for j, (e, _) in enumerate(picks):
            note("gate", close(st["gate"][t, j], mv(L.gate[0][e], L.gate[1][e], inter, h, x), f"t{t} e{e} gate"))
            note("up", close(st["up"][t, j], mv(L.up[0][e], L.up[1][e], inter, h, x), f"t{t} e{e} up"))
            hid = O.swiglu(st["gate"][t, j], st["up"][t, j])
            hq, hs_, _ = O.qact(hid)
            if m > 1:  # the device's own codes feed the down reference
                dq, ds = st["hidden_qs"][t, j], st["hidden_scales"][t, j]
                codes += dq.size
                flips += int(np.count_nonzero(dq != hq))
                assert np.all(np.abs(dq.astype(np.int32) - hq) <= 1), f"t{t} e{e}: a code off by more than one"
                hq, hs_ = dq, ds
            note("down", close(st["out"][t, j], mv_codes(L.down[0][e], L.down[1][e], h, inter, hq, hs_),
                               f"t{t} e{e} down"))
        v = np.zeros(h, np.float32)
        if L.sh:
            note("shared gate", close(st["shared_gate"][t], mv(*L.sg, L.sh, h, x), f"t{t} shared gate"))
            note("shared up", close(st["shared_up"][t], mv(*L.su, L.sh, h, x), f"t{t} shared up"))
            sq, ss, _ = O.qact(O.swiglu(st["shared_gate"][t], st["shared_up"][t]))
            note("shared down", close(st["shared_out"][t], mv_codes(*L.sd, h, L.sh, sq, ss), f"t{t} shared down"))
            v = st["shared_out"][t].copy()
        for j in range(n):  # mix: expert order, float32, as the device adds
            v = (v + (st["weights"][t, j] * st["out"][t, j]).astype(np.float32)).astype(np.float32)
        np.testing.assert_array_equal(out[t], v, err_msg=f"token {t}: mix")
    return worst, flips, codes


SMALL = dict(hidden=256, inter=128, n_exp=16, top_k=4, sh_inter=256)


@pytest.mark.parametrize("m", [1, 33])
def test_each_stage_of_a_small_layer(ctx, m):
    say("moe stages small", m)
    L = Layer(ctx, seed=900, **SMALL)
    hs = O.normal(901 + m, m * SMALL["hidden"])
    worst, flips, codes = check_stages(L, hs, m, range(m))
    say("moe stages small worst", m, {k: f"{v:.1e}" for k, v in worst.items()}, f"flips {flips}/{codes}")


@pytest.mark.parametrize("hidden", [4096, 8192])
def test_each_stage_with_wide_router_rows(ctx, hidden):
    # a batch's router logits come from one workgroup per token, one 32-block
    # of the row per lane: rows of 4096 and 8192 values take two and four
    # blocks a lane (and fewer rows in flight a wave)
    say("moe stages wide router rows", hidden)
    L = Layer(ctx, hidden=hidden, inter=64, n_exp=24, top_k=3, seed=930 + hidden // 1024)
    m = 7
    hs = O.normal(931, m * hidden)
    worst, flips, codes = check_stages(L, hs, m, range(m))
    say("moe stages wide worst", hidden, {k: f"{v:.1e}" for k, v in worst.items()}, f"flips {flips}/{codes}")


def test_each_stage_with_many_experts(ctx):
    # 160 experts (DeepSeek-V2's count): each wave of the per-token router
    # takes rows wave * 16 .. + 15 of every 64, three rounds, the last partial
    say("moe stages 160 experts")
    L = Layer(ctx, hidden=512, inter=32, n_exp=160, top_k=6, seed=940)
    m = 9
    hs = O.normal(941, m * 512)
    worst, flips, codes = check_stages(L, hs, m, range(m))
    say("moe stages 160 worst", {k: f"{v:.1e}" for k, v in worst.items()}, f"flips {flips}/{codes}")


@pytest.fixture(scope="module")
def deepseek(ctx):
    # hidden 2048, 64 routed experts of width 1408, top-6,
    # a fused shared expert of width 2816
    return Layer(ctx, hidden=2048, inter=1408, n_exp=64, top_k=6, seed=950, sh_inter=2816)


@pytest.mark.parametrize("m", [1, 512])
def test_each_stage_of_the_deepseek_v2_lite_layer(ctx, deepseek, m):
    say("moe stages deepseek", m)
    hs = O.normal(960 + m, m * 2048)
    tokens = range(m) if m == 1 else [0, 1, 100, 255, 256, 400, 510, 511]
    worst, flips, codes = check_stages(deepseek, hs, m, tokens)
    say("moe stages deepseek worst", m, {k: f"{v:.1e}" for k, v in worst.items()}, f"flips {flips}/{codes}")
    if m > 1:
        assert flips <= codes // 100, f"{flips} of {codes} hidden codes at a boundary"


def test_the_layer_bar_is_boundary_flips(ctx, deepseek):
    # Where the layer's output parts from the oracle's (test_gpu_moe.py holds
    # it to 2e-3): the oracle's own gate and up (f32 sums in its order) differ
    # from the device's in the last bits, so swiglu of them lands on the other
    # side of a quantisation boundary for a few hidden values -- each such
    # code is one step off, and there are no others.  The stages themselves
    # agree to 1e-5 (above).
    L, m = deepseek, 512
    hs = O.normal(960 + m, m * 2048)
    L.moe.run(hs, m)
    st = L.moe.picks(m, hidden_codes=True)
    flips = codes = 0
    for t in (3, 77, 300):
        x = hs[t * 2048:(t + 1) * 2048]
        for j in range(int(st["count"][t])):
            e = int(st["experts"][t, j])
            g = O.matvec_q8(L.gate[0][e], L.gate[1][e], L.inter, 2048, x)
            u = O.matvec_q8(L.up[0][e], L.up[1][e], L.inter, 2048, x)
            oq = O.qact(O.swiglu(g, u))[0]
            dq = st["hidden_qs"][t, j]
            assert np.all(np.abs(oq.astype(np.int32) - dq) <= 1)
            flips += int(np.count_nonzero(oq != dq))
            codes += dq.size
    say("moe oracle-chain hidden code flips", f"{flips}/{codes}")
    assert flips <= codes // 100

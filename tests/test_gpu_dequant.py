"""GPU parity of the dequantising GEMV (Weight::matvec_bt_dequant,
crates/llm/src/quant.rs:522-589) through the C ABI.

Bar: f32 outputs within 1e-5 x max|ref|.  q8 and q4 against the oracle's
restatement of the reference kernel (kvo_matvec_dequant, itself pinned
against float64 in test_oracle.py); Q4_K, which the reference's CPU engine
has no dequantising kernel for, against the float64 product of the
bit-exact dequantised rows (Weight::row / mpp.rs:304-315) with the f32
activation.  The KVAD_DEQUANT switch (quant.rs:592-610): kh_matvec runs the
same kernel, and matvec_many declines as the reference returns None.
"""
import os

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

import kvad_amd as K  # noqa: E402  (fails loudly without libkvad_hip.so)

RTOL = 1e-5


def close(got, want, rtol=RTOL):
    scale = max(float(np.max(np.abs(want))), 1e-30)
    err = float(np.max(np.abs(got.astype(np.float64) - want)))
    assert err <= rtol * scale, f"max err {err:.3e} vs scale {scale:.3e}"


def say(*a):
    print("[case]", *a, flush=True)


def make(ctx, prec, rows, cols, seed):
    w = O.normal(seed, rows * cols, 0.02)
    if prec == "q8":
        s, q = O.quantize_q8(w, rows, cols)
        return K.Weight.from_q8(ctx, rows, cols, s, q), (s, q)
    if prec == "q4":
        s, q = O.quantize_q4(w, rows, cols)
        return K.Weight.from_q4(ctx, rows, cols, s, q), (s, q)
    b = O.quantize_q4k(w, rows, cols)
    return K.Weight.from_q4k(ctx, rows, cols, b), (b,)


def reference(prec, parts, rows, cols, x, bias=None):
    if prec == "q8":
        y = O.matvec_dequant(1, parts[0], parts[1], rows, cols, x).astype(np.float64)
    elif prec == "q4":
        y = O.matvec_dequant(2, parts[0], parts[1], rows, cols, x).astype(np.float64)
    else:
        wd = np.stack([O.row_q4k(parts[0], cols, r) for r in range(rows)]).astype(np.float64)
        y = wd @ x.astype(np.float64)
    if bias is not None:
        y = (y.astype(np.float32) + bias).astype(np.float64)  # quant.rs:505-509: bias added after
    return y


SHAPES = {
    "q8": [(1, 32), (13, 64), (203, 96), (4864, 896), (896, 4864)],
    "q4": [(1, 32), (13, 64), (203, 96), (4864, 896), (896, 4864)],
    "q4k": [(1, 256), (13, 512), (64, 1024), (4096, 4096), (1024, 14336)],
}


@pytest.mark.parametrize("prec,shape", [(p, s) for p, ss in SHAPES.items() for s in ss])
def test_dequant_matvec_matches_the_reference(ctx, prec, shape):
    rows, cols = shape
    say("dequant", prec, rows, cols)
    W, parts = make(ctx, prec, rows, cols, 42 + rows)
    x = O.normal(7 + cols, cols)
    close(W.matvec_bt_dequant(x), reference(prec, parts, rows, cols, x))


@pytest.mark.parametrize("prec", ["q8", "q4", "q4k"])
def test_dequant_matvec_adds_the_bias(ctx, prec):
    rows, cols = (37, 512)
    say("dequant bias", prec)
    W, parts = make(ctx, prec, rows, cols, 5)
    x = O.normal(6, cols)
    bias = O.normal(9, rows)
    close(W.matvec_bt_dequant(x, bias), reference(prec, parts, rows, cols, x, bias))


def test_dequant_on_device_pointers_equals_the_host_call(ctx):
    import torch

    rows, cols = 4864, 896
    say("dequant dev", rows, cols)
    W, _ = make(ctx, "q8", rows, cols, 11)
    x = O.normal(12, cols)
    xd = torch.from_numpy(x).cuda()
    yd = torch.empty(rows, device="cuda")
    torch.cuda.synchronize()
    W.matvec_bt_dequant_dev(xd.data_ptr(), yd.data_ptr())
    ctx.synchronize()
    np.testing.assert_array_equal(yd.cpu().numpy(), W.matvec_bt_dequant(x))


def test_kvad_dequant_switch_selects_the_kernel(ctx):
    rows, cols = 896, 4864
    say("KVAD_DEQUANT", rows, cols)
    W, parts = make(ctx, "q8", rows, cols, 21)
    x = O.normal(22, cols)
    integer = W.matvec_bt(x)
    dq = W.matvec_bt_dequant(x)
    old = os.environ.get("KVAD_DEQUANT")
    try:
        os.environ["KVAD_DEQUANT"] = "1"
        np.testing.assert_array_equal(W.matvec_bt(x), dq)
        # quant.rs:629-633: matvec_many returns None under the switch
        assert K.matvec_many(ctx, [(W, x), (W, x)]) is None
        os.environ["KVAD_DEQUANT"] = "true"
        np.testing.assert_array_equal(W.matvec_bt(x), dq)
        os.environ["KVAD_DEQUANT"] = "0"
        np.testing.assert_array_equal(W.matvec_bt(x), integer)
    finally:
        if old is None:
            os.environ.pop("KVAD_DEQUANT", None)
        else:
            os.environ["KVAD_DEQUANT"] = old
    np.testing.assert_array_equal(W.matvec_bt(x), integer)
    # the two kernels agree to the quantisation of x (quant.rs:1190-1208 bounds)
    close(dq, O.matvec_q8(*parts, rows, cols, x).astype(np.float64), rtol=0.03)


def test_dequant_rejects_f32_weights(ctx):
    W = K.Weight.from_f32(ctx, np.ones((4, 32), np.float32))
    with pytest.raises(K.KvadError):
        W.matvec_bt_dequant(np.ones(32, np.float32))

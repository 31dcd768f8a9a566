"""GPU parity of the decode glue -- RMSNorm, RoPE, SwiGLU, softmax
(tensor.rs:297-472) -- against the oracle, through the C ABI on device
arrays (torch holds the device memory).

Bar: RoPE bit-exact (the caller's tables, the reference's two products and
one sum); RMSNorm and softmax within 1e-5 x max|ref| (a tree sum against the
reference's serial one); SwiGLU within 1e-6 relative (the device's exp).
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

import kvad_amd as K  # noqa: E402

torch = pytest.importorskip("torch")

from test_gpu_gemv import close, say  # noqa: E402


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.fixture()
def dctx(ctx):
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    yield ctx
    ctx.set_stream(None)


@pytest.mark.parametrize("n", [64, 896, 2048, 4096])
def test_rms_norm(dctx, n):
    say("rms_norm", n)
    m = 3
    x = O.normal(n, m * n)
    w = O.normal(n + 1, n)
    out = torch.empty(m * n, device="cuda")
    dx, dw = dev(x), dev(w)
    K.rms_norm_dev(dctx, dx.data_ptr(), dw.data_ptr(), m, n, 1e-6, out.data_ptr())
    got = host(out)
    for r in range(m):
        close(got[r * n:(r + 1) * n], O.rms_norm(x[r * n:(r + 1) * n], w, 1e-6))


@pytest.mark.parametrize("interleaved", [False, True])
def test_rope_is_bit_exact(dctx, interleaved):
    say("rope", interleaved)
    hd, n_vec, m, pos0 = 64, 14, 5, 3
    c, s = O.rope_tables(hd, 64, 1e6)
    x = O.normal(9, m * n_vec * hd)
    dx, dc, ds = dev(x), dev(c), dev(s)  # held: a freed temporary's block is reused at once
    K.rope_dev(dctx, dc.data_ptr(), ds.data_ptr(), hd // 2, dx.data_ptr(), m, n_vec, pos0, interleaved)
    got = host(dx)
    fn = O.rope_apply_interleaved if interleaved else O.rope_apply
    want = np.concatenate([fn(c, s, hd // 2, x[(r * n_vec + v) * hd:(r * n_vec + v + 1) * hd], pos0 + r)
                           for r in range(m) for v in range(n_vec)])
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_swiglu(dctx):
    say("swiglu")
    n = 4864
    g, u = O.normal(1, n) * 4.0, O.normal(2, n)
    dg, du = dev(g), dev(u)
    K.swiglu_dev(dctx, dg.data_ptr(), du.data_ptr(), n)
    np.testing.assert_allclose(host(dg), O.swiglu(g, u), rtol=1e-6, atol=1e-30)


@pytest.mark.parametrize("n", [8, 64, 1000])
def test_softmax(dctx, n):
    say("softmax", n)
    m = 4
    x = O.normal(n, m * n) * 20.0
    dx = dev(x)
    K.softmax_dev(dctx, dx.data_ptr(), m, n)
    got = host(dx)
    for r in range(m):
        close(got[r * n:(r + 1) * n], O.softmax(x[r * n:(r + 1) * n]))
        assert abs(float(got[r * n:(r + 1) * n].sum()) - 1.0) < 1e-5

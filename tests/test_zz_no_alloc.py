"""The attention entry point that allocates nothing (kh_attend_dev_noalloc):
its output equals kh_attend_dev's, bit for bit, on two calls in a row, the
second with a smaller input; a call whose partials exceed the library's
static scratch array is refused with a clear error."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

import kvad_amd as K  # noqa: E402


def say(*a):
    print("[case]", *a, flush=True)


def run(ctx, fn, n_head, n_kv, hd, q, k, v, L, out):
    rc = fn(ctx.h, n_head, n_kv, hd, q.data_ptr(), k.data_ptr(), v.data_ptr(), L, out.data_ptr())
    return rc


@pytest.mark.parametrize("geom,lengths", [((14, 2, 64), (8192, 1000)), ((32, 8, 128), (4096, 300)),
                                          ((14, 2, 64), (32768, 1))])
def test_noalloc_attention_equals_the_allocating_entry(ctx, geom, lengths):
    import torch

    n_head, n_kv, hd = geom
    kv_dim = n_kv * hd
    g = torch.Generator(device="cuda")
    g.manual_seed(1234)
    Lmax = max(lengths)
    k = torch.randn(Lmax, kv_dim, device="cuda", generator=g)
    v = torch.randn(Lmax, kv_dim, device="cuda", generator=g)
    for L in lengths:  # the second call is smaller than the first
        say("noalloc", geom, L)
        q = torch.randn(n_head * hd, device="cuda", generator=g)
        want = torch.empty(n_head * hd, device="cuda")
        got = torch.full((n_head * hd,), float("nan"), device="cuda")
        torch.cuda.synchronize()
        assert run(ctx, K.lib.kh_attend_dev, n_head, n_kv, hd, q, k, v, L, want) == 0, K.lib.kh_last_error()
        assert run(ctx, K.lib.kh_attend_dev_noalloc, n_head, n_kv, hd, q, k, v, L, got) == 0, K.lib.kh_last_error()
        ctx.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy())


def test_noalloc_attention_of_no_positions_is_zero(ctx):
    import torch

    say("noalloc L=0")
    q = torch.randn(14 * 64, device="cuda")
    out = torch.full((14 * 64,), 7.0, device="cuda")
    torch.cuda.synchronize()
    assert K.lib.kh_attend_dev_noalloc(ctx.h, 14, 2, 64, q.data_ptr(), None, None, 0, out.data_ptr()) == 0
    ctx.synchronize()
    assert not out.cpu().numpy().any()


def test_noalloc_attention_refuses_what_exceeds_the_scratch(ctx):
    import torch

    assert K.lib.kh_noalloc_scratch_bytes() == 8 << 20
    # 64 heads of 128 over 32768 positions: 128 splits x 64 heads of partials (12.7 MB)
    n_head, n_kv, hd, L = 64, 8, 128, 32768
    say("noalloc too large", n_head, L)
    k = torch.zeros(L, n_kv * hd, device="cuda")
    v = torch.zeros(L, n_kv * hd, device="cuda")
    q = torch.zeros(n_head * hd, device="cuda")
    out = torch.empty(n_head * hd, device="cuda")
    torch.cuda.synchronize()
    rc = run(ctx, K.lib.kh_attend_dev_noalloc, n_head, n_kv, hd, q, k, v, L, out)
    assert rc == -1  # KH_EINVAL
    assert b"bytes of scratch" in K.lib.kh_last_error()

"""Absorbed latent attention on the device (kh_mla_attend, model/deepseek.rs:553-591)
against the oracle: the cache is the reference's (keys = rotated pe rows of 64,
values = latents of 512), every head scores the same rows.  Tolerance 1e-4 of
the output's largest magnitude, the attention bar; one position is exact."""
import numpy as np
import pytest

import kvad_amd as K
import oracle as O

pytestmark = pytest.mark.gpu
SCALE = 1.0 / np.sqrt(192.0)  # DeepSeek-V2-Lite: 1 / sqrt(qk_nope + qk_rope)


def _case(seed, H, L):
    rng = np.random.default_rng(seed)
    ql = rng.standard_normal((H, 512)).astype(np.float32)
    qp = rng.standard_normal((H, 64)).astype(np.float32)
    c = rng.standard_normal((L, 512)).astype(np.float32)
    pe = rng.standard_normal((L, 64)).astype(np.float32)
    return ql, qp, c, pe


def _run(ctx, ql, qp, c, pe, H, L):
    cache = K.KvCache(ctx, 1, 64, 512)
    cache.push(0, pe.ravel(), c.ravel())
    return K.mla_attend(ctx, cache, 0, H, ql, qp, L, SCALE).reshape(H, 512)


@pytest.mark.parametrize("H, L", [(16, 1), (16, 3), (16, 64), (16, 65), (16, 200), (16, 1000), (16, 5000),
                                  (8, 130), (20, 333)])
def test_latent_attention_matches_the_oracle(ctx, H, L):
    ql, qp, c, pe = _case(H * 7919 + L, H, L)
    got = _run(ctx, ql, qp, c, pe, H, L)
    want = O.mla_attend(H, 512, 64, ql, qp, c, pe, L, SCALE).reshape(H, 512)
    err = np.max(np.abs(got - want))
    assert err <= 1e-4 * np.max(np.abs(want)), (H, L, err)
    if L == 1:
        assert np.array_equal(got, want)


@pytest.mark.parametrize("L", [40, 300])  # one split (the kernel's own weights), several (the merge's correction)
def test_weights_below_1e_8_are_dropped(ctx, L):
    H = 16
    ql, qp, c, pe = _case(L, H, L)
    qp[:] = 0.0
    for t in (7, L - 3):
        c[t] = -ql[t % H] * 3.0  # far below the rest for one head
    got = _run(ctx, ql, qp, c, pe, H, L)
    want = O.mla_attend(H, 512, 64, ql, qp, c, pe, L, SCALE).reshape(H, 512)
    assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want))


def test_device_pointer_entry(ctx):
    import torch

    H, L = 16, 777
    ql, qp, c, pe = _case(3, H, L)
    dev = torch.device("cuda:0")
    t = {k: torch.from_numpy(v.copy()).to(dev) for k, v in dict(ql=ql, qp=qp, c=c, pe=pe).items()}
    out = torch.empty(H * 512, device=dev)
    K.mla_attend_dev(ctx, H, t["ql"].data_ptr(), t["qp"].data_ptr(), t["c"].data_ptr(), t["pe"].data_ptr(), L,
                     SCALE, out.data_ptr())
    torch.cuda.synchronize()
    want = O.mla_attend(H, 512, 64, ql, qp, c, pe, L, SCALE)
    assert np.max(np.abs(out.cpu().numpy() - want)) <= 1e-4 * np.max(np.abs(want))


def test_a_cache_of_other_widths_is_declined(ctx):
    cache = K.KvCache(ctx, 1, 128, 128)
    cache.push(0, np.zeros(128, np.float32), np.zeros(128, np.float32))
    with pytest.raises(K.Declined):
        K.mla_attend(ctx, cache, 0, 16, np.zeros(16 * 512), np.zeros(16 * 64), 1, SCALE)


@pytest.mark.parametrize("L", [3000, 20000])
def test_skip_across_many_splits(ctx, L):
    # dominant positions and a spread across the 1e-8 line (see test_gpu_attend)
    H = 16
    rng = np.random.default_rng(L + 1)
    ql = np.zeros((H, 512), np.float32)
    qp = np.zeros((H, 64), np.float32)
    qp[:, 0] = np.sqrt(192.0)  # score_t = pe_t[0]
    c = (rng.standard_normal((L, 512)) * 100.0).astype(np.float32)
    pe = np.zeros((L, 64), np.float32)
    pe[:, 0] = rng.uniform(-4.0, 10.0, L)
    pe[rng.choice(L, 3, replace=False), 0] = 24.0
    got = _run(ctx, ql, qp, c, pe, H, L)
    want = O.mla_attend(H, 512, 64, ql, qp, c, pe, L, SCALE).reshape(H, 512)
    assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want))


@pytest.mark.parametrize("dims", ["32", "64", "128"])
def test_every_merge_width_matches_the_oracle(ctx, monkeypatch, dims):
    # the merge cut into 32-, 64- or 128-dim workgroups per head, over many
    # splits: random rows, and dominant positions with a spread across the
    # 1e-8 line (as test_skip_across_many_splits builds them)
    monkeypatch.setenv("KVAD_MLA_MERGE_D", dims)
    H, L = 16, 4500
    ql, qp, c, pe = _case(H * 31 + L, H, L)
    got = _run(ctx, ql, qp, c, pe, H, L)
    want = O.mla_attend(H, 512, 64, ql, qp, c, pe, L, SCALE).reshape(H, 512)
    assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want)), (dims, "random")
    rng = np.random.default_rng(L + 7)
    ql = np.zeros((H, 512), np.float32)
    qp = np.zeros((H, 64), np.float32)
    qp[:, 0] = np.sqrt(192.0)  # score_t = pe_t[0]
    c = (rng.standard_normal((L, 512)) * 100.0).astype(np.float32)
    pe = np.zeros((L, 64), np.float32)
    pe[:, 0] = rng.uniform(-4.0, 10.0, L)
    pe[rng.choice(L, 3, replace=False), 0] = 24.0
    got = _run(ctx, ql, qp, c, pe, H, L)
    want = O.mla_attend(H, 512, 64, ql, qp, c, pe, L, SCALE).reshape(H, 512)
    assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want)), (dims, "skip")


@pytest.mark.parametrize("L", [1, 100, 129, 3000])
def test_128_position_splits_match_the_oracle(ctx, monkeypatch, L):
    # eight-wave splits of 128 positions (taken on their own past 32768
    # positions): one split, a ragged last split, and the 1e-8 skip across
    # many splits
    monkeypatch.setenv("KVAD_MLA_SPLIT", "128")
    H = 16
    ql, qp, c, pe = _case(H * 13 + L, H, L)
    if L == 3000:
        rng = np.random.default_rng(L + 11)
        ql = np.zeros((H, 512), np.float32)
        qp = np.zeros((H, 64), np.float32)
        qp[:, 0] = np.sqrt(192.0)  # score_t = pe_t[0]
        c = (rng.standard_normal((L, 512)) * 100.0).astype(np.float32)
        pe = np.zeros((L, 64), np.float32)
        pe[:, 0] = rng.uniform(-4.0, 10.0, L)
        pe[rng.choice(L, 3, replace=False), 0] = 24.0
    got = _run(ctx, ql, qp, c, pe, H, L)
    want = O.mla_attend(H, 512, 64, ql, qp, c, pe, L, SCALE).reshape(H, 512)
    assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want)), L

"""GPU parity of decode attention and the device KV cache against the oracle.

Bar: within 1e-4 x max|ref| (the reference's own agreement bar between
attention variants, examples/bench_attend.rs:111-115); exact at one
position, where every weight is 1.
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

import kvad_amd as K  # noqa: E402

QWEN = K.Spec(14, 2, 64)
LLAMA = K.Spec(32, 8, 128)


def say(*a):
    print("[case]", *a, flush=True)


def close(got, want, rtol=1e-4):
    scale = max(float(np.max(np.abs(want))), 1e-3)
    err = float(np.max(np.abs(got.astype(np.float64) - want)))
    assert err <= rtol * scale, f"max err {err:.3e} vs scale {scale:.3e}"


def filled_cache(ctx, spec, L, seed, layers=1):
    cache = K.KvCache(ctx, layers, spec.kv_dim, spec.kv_dim)
    ks, vs = [], []
    for l in range(layers):
        k = O.normal(seed + 2 * l, L * spec.kv_dim)
        v = O.normal(seed + 2 * l + 1, L * spec.kv_dim)
        cache.push(l, k, v)
        ks.append(k)
        vs.append(v)
    cache.len = L
    return cache, ks, vs


@pytest.mark.parametrize("spec,L", [(QWEN, 1), (QWEN, 2), (QWEN, 17), (QWEN, 1024), (QWEN, 8192), (QWEN, 32768),
                                    (LLAMA, 1), (LLAMA, 513), (LLAMA, 2048), (K.Spec(4, 4, 64), 100),
                                    (K.Spec(16, 1, 128), 300), (K.Spec(24, 2, 64), 77)])
def test_attend_matches_the_oracle(ctx, spec, L):
    say("attend", spec, L)
    cache, ks, vs = filled_cache(ctx, spec, L, seed=L)
    q = O.normal(L + 100, spec.n_head * spec.head_dim)
    got = K.attend(ctx, spec, q, cache, 0, L)
    want = O.attend(spec.n_head, spec.n_kv_head, spec.head_dim, q, ks[0], vs[0], L)
    close(got, want)
    if L == 1:
        np.testing.assert_array_equal(got, want)


def test_attend_over_a_prefix_of_the_cache(ctx):
    # causal prefill reads n_positions < len (llama.rs:258-271)
    say("attend prefix")
    cache, ks, vs = filled_cache(ctx, QWEN, 500, seed=9)
    q = O.normal(10, 14 * 64)
    for n in (1, 100, 499, 500):
        got = K.attend(ctx, QWEN, q, cache, 0, n)
        close(got, O.attend(14, 2, 64, q, ks[0], vs[0], n))


def test_attend_skips_weights_below_1e8(ctx):
    # model/mod.rs:807
    say("attend skip")
    spec = K.Spec(1, 1, 64)
    L = 40
    q = np.zeros(64, np.float32)
    q[0] = 10.0
    k = np.zeros(L * 64, np.float32)
    k[0] = 80.0
    v = np.full(L * 64, 1e6, np.float32)
    v[:64] = 1.0
    cache = K.KvCache(ctx, 1, 64, 64)
    cache.push(0, k, v)
    got = K.attend(ctx, spec, q, cache, 0, L)
    np.testing.assert_array_equal(got, O.attend(1, 1, 64, q, k, v, L))


def test_attend_is_deterministic(ctx):
    say("attend determinism")
    cache, _, _ = filled_cache(ctx, QWEN, 4096, seed=3)
    q = O.normal(4, 14 * 64)
    first = K.attend(ctx, QWEN, q, cache, 0, 4096)
    for _ in range(4):
        np.testing.assert_array_equal(K.attend(ctx, QWEN, q, cache, 0, 4096), first)


def test_zero_positions_give_zeros(ctx):
    say("attend empty")
    cache = K.KvCache(ctx, 1, 128, 128)
    out = K.attend(ctx, QWEN, O.normal(1, 14 * 64), cache, 0, 0)
    assert np.all(out == 0)


def test_cache_push_grows_and_keeps_every_row(ctx):
    # KvCache::push appends (mod.rs:666-669); the device cache doubles from 256
    say("kv grow")
    cache = K.KvCache(ctx, 2, 128, 128, capacity=4)
    rows_k, rows_v = [], []
    for step in range(40):
        k = O.normal(step, 128)
        v = O.normal(step + 1000, 128)
        for l in range(2):
            cache.push(l, k + l, v - l)
        rows_k.append(k)
        rows_v.append(v)
        cache.len = cache.len + 1
    assert cache.len == 40
    np.testing.assert_array_equal(cache.keys(1), (np.concatenate(rows_k) + 1).astype(np.float32))
    np.testing.assert_array_equal(cache.values(0), np.concatenate(rows_v))


def test_truncation_keeps_the_prefix(ctx):
    # mod.rs:1299-1322 restated: truncating keeps the first len rows, and
    # never extends
    say("kv truncate")
    cache, ks, vs = filled_cache(ctx, QWEN, 50, seed=1, layers=3)
    assert cache.truncate(60) == 50
    assert cache.truncate(20) == 20
    assert cache.len == 20
    for l in range(3):
        np.testing.assert_array_equal(cache.keys(l), ks[l][:20 * 128])
        np.testing.assert_array_equal(cache.values(l), vs[l][:20 * 128])
    cache.clear()
    assert cache.len == 0 and cache.keys(0).size == 0


def test_attend_rejects_more_positions_than_cached(ctx):
    say("attend errors")
    cache, _, _ = filled_cache(ctx, QWEN, 10, seed=1)
    with pytest.raises(K.KvadError):
        K.attend(ctx, QWEN, O.normal(1, 14 * 64), cache, 0, 11)
    with pytest.raises(K.KvadError):
        K.attend(ctx, K.Spec(14, 3, 64), O.normal(1, 14 * 64), cache, 0, 5)


# KVAD_ATTN_SINGLE lowers the longest sequence taken as one split (256
# positions at head_dim 64, 128 at 128): 0 makes every call split and merge.
SINGLE, SPLIT = None, "0"


def attn_mode(monkeypatch, mode):
    if mode is None:
        monkeypatch.delenv("KVAD_ATTN_SINGLE", raising=False)
    else:
        monkeypatch.setenv("KVAD_ATTN_SINGLE", mode)


@pytest.mark.parametrize("spec,L", [(QWEN, 1), (QWEN, 17), (QWEN, 100), (QWEN, 200), (QWEN, 256), (LLAMA, 1),
                                    (LLAMA, 100), (LLAMA, 128), (K.Spec(16, 1, 128), 128),
                                    (K.Spec(4, 4, 64), 233), (K.Spec(24, 2, 64), 77)])
def test_one_split_and_split_merge_agree(ctx, monkeypatch, spec, L):
    # the whole sequence as one split (the reference's exact weights, no
    # merge launch) against the same call split and merged, both against
    # the oracle; at one position both are exact
    say("attend single vs split", spec, L)
    cache, ks, vs = filled_cache(ctx, spec, L, seed=L + 5)
    q = O.normal(L + 105, spec.n_head * spec.head_dim)
    want = O.attend(spec.n_head, spec.n_kv_head, spec.head_dim, q, ks[0], vs[0], L)
    attn_mode(monkeypatch, SINGLE)
    single = K.attend(ctx, spec, q, cache, 0, L)
    attn_mode(monkeypatch, SPLIT)
    split = K.attend(ctx, spec, q, cache, 0, L)
    close(single, want)
    close(split, want)
    if L == 1:
        np.testing.assert_array_equal(single, want)
        np.testing.assert_array_equal(split, want)


@pytest.mark.parametrize("n_head,n_kv,L,mode", [(4, 1, 3000, SPLIT), (4, 1, 20000, SPLIT), (14, 2, 32768, SPLIT),
                                                (14, 2, 1000, SPLIT), (4, 1, 256, SPLIT), (4, 1, 256, SINGLE),
                                                (14, 2, 250, SINGLE), (16, 1, 200, SINGLE)])
def test_attend_skip_across_many_splits(ctx, monkeypatch, n_head, n_kv, L, mode):
    # A few dominant positions; the rest spread across the 1e-8 line, so some
    # splits are left out whole, some kept whole and most straddle it.  Values
    # are large, so a skipped term wrongly kept (or a kept one dropped) shows.
    # Qwen's geometry at 32768 positions runs the 256-position splits, at
    # 1000 the two-wave 32-position ones; a single split drops the same
    # weights itself.
    attn_mode(monkeypatch, mode)
    say("attend skip, many splits", n_head, n_kv, L, mode)
    spec = K.Spec(n_head, n_kv, 64)
    kvd = n_kv * 64
    rng = np.random.default_rng(L)
    q = np.zeros((n_head, 64), np.float32)
    q[:, 0] = 8.0  # score_t = q . k_t / 8 = k_t[0] of the head's KV head
    k = np.zeros((L, kvd), np.float32)
    for h in range(n_kv):
        k[:, 64 * h] = rng.uniform(-4.0, 10.0, L)
        k[rng.choice(L, 3, replace=False), 64 * h] = 24.0
    v = (rng.standard_normal((L, kvd)) * 100.0).astype(np.float32)
    cache = K.KvCache(ctx, 1, kvd, kvd)
    cache.push(0, k.ravel(), v.ravel())
    got = K.attend(ctx, spec, q.ravel(), cache, 0, L)
    want = O.attend(n_head, n_kv, 64, q.ravel(), k.ravel(), v.ravel(), L)
    close(got, want)

"""xtg_hip_attention_noalloc (include/xtg_hip.h): the attention call that allocates nothing, its split partials in the
device's fixed scratch array, against xtg_hip_attention (the same kernels on scratch the backend allocates) through
the C ABI. Bar: equal bit for bit (integer-exact agreement is expected: the same kernels, plan and summation order).

- Two calls in a row, the second smaller (a global cache at a 4K context with an 8-row verify step, then a 1088-slot
  ring read by one row), so the second runs on what the first left in the shared array; FP8 caches as well.
- A fresh backend, whose own attention scratch was never sized, captures the call into a HIP graph and replays it
  (first in this file: the array then belongs to that backend until it is closed).
- A call whose partials exceed the array is refused before anything is queued; so is a call from a second open
  backend on the device while the first holds the array (their calls would race on it).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HEADS, KVH, D = 32, 8, 128


def unit(rng, shape):
    x = rng.standard_normal(shape).astype(np.float32)
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def make_case(b, rng, ctx, n_q, ring=0, dtype=0):
    """A cache holding positions 0 .. ctx - 1 (a ring: the last `ring` of them), and the call's q, k, v, out."""
    cache = b.kv_cache(KVH, D, ctx + n_q, ring=ring, dtype=dtype)
    lo = max(0, ctx - ring) if ring else 0
    K = unit(rng, (ctx - lo, KVH, D))
    V = unit(rng, (ctx - lo, KVH, D))
    for p in range(lo, ctx, 2048):
        q = min(ctx, p + 2048)
        cache.store_host(p, K[p - lo:q - lo], V[p - lo:q - lo])
    arrays = [b.array(unit(rng, (n_q, HEADS, D))), b.array(unit(rng, (n_q, KVH, D))),
              b.array(unit(rng, (n_q, KVH, D))), b.array(shape=(n_q, HEADS, D))]
    return cache, arrays


def run(b, fn, case, ctx, n_q, window):
    cache, (q, k, v, out) = case
    out.upload(np.full((n_q, HEADS, D), np.nan, np.float32))
    fn(cache, q, k, v, out, n_q, ctx, HEADS, window=window)
    return out.numpy()


def test_noalloc_under_graph_capture(pkg):
    b = pkg.HipBackend(0)   # its attention scratch has never been sized; it holds the device's array until closed
    try:
        rng = np.random.default_rng(701)
        case = make_case(b, rng, 2048, 8)
        cache, (q, k, v, out) = case
        b.graph_begin()
        b.attention_noalloc(cache, q, k, v, out, 8, 2048, HEADS)
        g = b.graph_end("attention_noalloc")
        want = run(b, b.attention, case, 2048, 8, 0)   # eager, on scratch the backend allocates now
        for rep in range(3):
            out.upload(np.full((8, HEADS, D), np.nan, np.float32))
            b.graph_launch(g)
            np.testing.assert_array_equal(out.numpy(), want)
            run(b, b.attention, case, 2048, 8, 0)   # eager work between replays
        b.graph_destroy(g)
        cache.destroy()
        for a in case[1]:
            a.free()
    finally:
        b.close()


@pytest.mark.parametrize("dtype", [0, 1])
def test_noalloc_matches_attention_two_calls(hip, dtype):
    rng = np.random.default_rng(700 + dtype)
    big = make_case(hip, rng, 4096, 8, dtype=dtype)
    small = make_case(hip, rng, 40000, 1, ring=1088, dtype=dtype)
    got_big = run(hip, hip.attention_noalloc, big, 4096, 8, 0)
    got_small = run(hip, hip.attention_noalloc, small, 40000, 1, 1024)   # right after, on the same array
    want_big = run(hip, hip.attention, big, 4096, 8, 0)
    want_small = run(hip, hip.attention, small, 40000, 1, 1024)
    assert np.isfinite(got_big).all() and np.isfinite(got_small).all()
    np.testing.assert_array_equal(got_big, want_big)
    np.testing.assert_array_equal(got_small, want_small)
    for cache, arrays in (big, small):
        cache.destroy()
        for a in arrays:
            a.free()


def test_noalloc_refuses_more_than_its_scratch(hip, pkg):
    """512 rows over 8 KV heads of 128 (64 row blocks, one key split and four own-key chunks) need about 43 MB of
    partials: more than the 16 MiB array."""
    rng = np.random.default_rng(702)
    cache, (q, k, v, out) = make_case(hip, rng, 4096, 512)
    with pytest.raises(pkg.XtgError, match="fixed scratch holds"):
        hip.attention_noalloc(cache, q, k, v, out, 512, 4096, HEADS)
    hip.finish()
    cache.destroy()
    for a in (q, k, v, out):
        a.free()


def test_noalloc_refuses_a_second_backend(hip, pkg):
    """While the session's backend holds the device's array (its call claims it), a second open backend's call is
    refused before anything is queued; the holder's calls still run and match xtg_hip_attention."""
    rng = np.random.default_rng(703)
    mine = make_case(hip, rng, 1024, 1)
    got = run(hip, hip.attention_noalloc, mine, 1024, 1, 0)
    b = pkg.HipBackend(0)
    try:
        other = make_case(b, rng, 1024, 1)
        cache, (q, k, v, out) = other
        with pytest.raises(pkg.XtgError, match="another open backend"):
            b.attention_noalloc(cache, q, k, v, out, 1, 1024, HEADS)
        np.testing.assert_array_equal(run(hip, hip.attention_noalloc, mine, 1024, 1, 0), got)
        np.testing.assert_array_equal(run(hip, hip.attention, mine, 1024, 1, 0), got)
        cache.destroy()
        for a in other[1]:
            a.free()
    finally:
        b.close()
    for c, arrays in (mine,):
        c.destroy()
        for a in arrays:
            a.free()

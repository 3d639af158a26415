"""GPU parity of the decode-step row kernels against the oracle (engine/src/kernels.cpp:162-234,
packs/dory/dory.cpp:474-475, :482-490, :510-515, :532-541). Bar: rel-L2 <= 1e-6 (single FP32 row passes)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def rel_l2(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(np.asarray(y, np.float64) - ref) / np.linalg.norm(ref))


@pytest.mark.parametrize("m,pos0", [(1, 0), (1, 4095), (8, 40000), (3, 123456)])
def test_qk_rope_norm(hip, orc, m, pos0):
    rng = np.random.default_rng(m + pos0)
    heads, kvh, d = 32, 8, 128
    q = rng.standard_normal((m, heads, d)).astype(np.float32)
    k = rng.standard_normal((m, kvh, d)).astype(np.float32)
    qs = rng.uniform(0.5, 1.5, heads * d).astype(np.float32)
    qo, ko = orc.qk_produce(q, k, heads, kvh, d, pos0, 1e6, qs)
    dq, dk, ds = hip.array(q), hip.array(k), hip.array(qs)
    hip.qk_rope_norm(dq, dk, m, heads, kvh, d, pos0, 1e6, ds)
    assert rel_l2(dq.numpy(), qo) <= 1e-6
    assert rel_l2(dk.numpy(), ko) <= 1e-6
    # no scale: q only normalised
    dq2 = hip.array(q)
    hip.qk_rope_norm(dq2, dk, m, heads, kvh, d, pos0, 1e4, None)
    qo2, _ = orc.qk_produce(q, k, heads, kvh, d, pos0, 1e4, np.ones(heads * d, np.float32))
    assert rel_l2(dq2.numpy(), qo2) <= 1e-6
    for a in (dq, dk, ds, dq2):
        a.free()


@pytest.mark.parametrize("rows,w", [(1, 3072), (8, 3072), (2, 4096)])
def test_slerp(hip, orc, rows, w):
    rng = np.random.default_rng(rows * w)
    x = rng.standard_normal((rows, w)).astype(np.float32)
    o = rng.standard_normal((rows, w)).astype(np.float32)
    lr = np.abs(rng.standard_normal(w)).astype(np.float32) * 0.05
    dx, do, dl = hip.array(x), hip.array(o), hip.array(lr)
    hip.slerp_residual(dx, do, dl, rows, w)
    assert rel_l2(dx.numpy(), orc.slerp_residual(x, o, lr)) <= 1e-6
    for a in (dx, do, dl):
        a.free()


@pytest.mark.parametrize("rows", [1, 8])
def test_swiglu_norm(hip, orc, rows):
    rng = np.random.default_rng(rows)
    w = 8192
    g = rng.standard_normal((rows, w)).astype(np.float32)
    u = rng.standard_normal((rows, w)).astype(np.float32)
    sg = rng.uniform(0.5, 1.5, w).astype(np.float32) * 50
    su = rng.uniform(0.5, 1.5, w).astype(np.float32) * 50
    dg, du, dsg, dsu = hip.array(g), hip.array(u), hip.array(sg), hip.array(su)
    hip.swiglu_norm(dg, du, dsg, dsu, rows, w)
    ref = orc.justnorm(orc.swiglu_scaled(g, u, sg, su))
    assert rel_l2(dg.numpy(), ref) <= 1e-6
    for a in (dg, du, dsg, dsu):
        a.free()


@pytest.mark.parametrize("rows", [1, 8])
def test_gate_and_add_norm(hip, orc, rows):
    rng = np.random.default_rng(10 + rows)
    w = 4096
    att = rng.standard_normal((rows, w)).astype(np.float32)
    gate = rng.standard_normal((rows, w)).astype(np.float32)
    gs = rng.uniform(0.5, 1.5, w).astype(np.float32) * 8
    da, dgt, dgs = hip.array(att), hip.array(gate), hip.array(gs)
    hip.gate_norm(da, dgt, dgs, rows, w)
    assert rel_l2(da.numpy(), orc.gate_norm(att, gate, gs)) <= 1e-6
    a = rng.standard_normal((rows, 3072)).astype(np.float32)
    b = rng.standard_normal((rows, 3072)).astype(np.float32)
    dx, dy, dz = hip.array(a), hip.array(b), hip.array(shape=(rows, 3072))
    hip.add_norm(dx, dy, dz, rows, 3072)
    assert rel_l2(dz.numpy(), orc.add_norm(a, b)) <= 1e-6
    hip.add_norm(dx, None, dx, rows, 3072)   # in place, no addend
    assert rel_l2(dx.numpy(), orc.add_norm(a)) <= 1e-6
    for arr in (da, dgt, dgs, dx, dy, dz):
        arr.free()


@pytest.mark.parametrize("rows,n", [(1, 131072), (8, 131072), (3, 1001), (2, 1), (4, 4096)])
def test_argmax(hip, orc, rows, n):
    """Greedy decoding's token per row (xtg::argmax, sampler.cpp:8-13), equal to the oracle's: rounded values (many
    ties, first index wins), a planted pair of equal maxima, NaN at element 0 (answer 0), NaNs elsewhere (passed
    over), a row of -inf (answer 0)."""
    rng = np.random.default_rng(rows * 7 + n)
    x = np.round(rng.standard_normal((rows, n)) * 4).astype(np.float32)
    if n > 10:
        x[0, n // 3] = x[0, n - 2] = x[0].max() + 1
    if rows > 1:
        x[1, 0] = np.nan
    if rows > 2:
        x[2, ::5] = np.nan
    if rows > 3:
        x[3] = -np.inf
    dx = hip.array(x)
    dout = hip.array(shape=(rows,), dtype=np.int32)
    hip.argmax(dx, rows, n, dout)
    got = dout.numpy()
    dx.free()
    dout.free()
    np.testing.assert_array_equal(got, orc.argmax(x))


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 37, 1000, 5000, 131072, 150001])
def test_sample(hip, orc, n):
    """xtg::Sampler::sample (sampler.cpp:40-94) on the device with the same draws as the oracle (itself pinned
    against the reference's Sampler): every filter combination over 8 rows at a time, greedy rows routed to argmax;
    ties planted among the most likely, and logits on a grid of 1/4 (exact ties through the kept candidates, which
    must come out in index order); top_k up to the slices' 64 listed weights (the union's first 64 only), just past
    them, past the 4096 the union holds (the whole row sorted), and the whole row; a row of 150001 (more than 4096
    listed weights, not a multiple of 4). The weights are FP32 exp values on both sides, so a token may differ only
    where r (or the top_p target) lies within a rounding step of a running-sum boundary: a mismatch counts as one
    only if the oracle's margin there exceeds 1e-6 of the total."""
    rng = np.random.default_rng(n)
    dout = hip.array(shape=(8,), dtype=np.int32)
    checked = 0
    for trial in range(24):
        rows = int(rng.integers(1, 9))
        x = (rng.standard_normal((rows, n)) * rng.choice([0.5, 2.0, 8.0])).astype(np.float32)
        if trial % 3 == 0 and n > 3:
            x[0, rng.integers(0, n, 3)] = x[0].max()   # ties among the most likely
        if trial % 4 == 1:
            x = np.round(x * 4) / 4   # ties everywhere
        params = dict(temperature=float(rng.choice([0.0, 0.3, 1.0, 2.0])),
                      top_p=float(rng.choice([1.0, 0.9, 0.5, 0.05])),
                      top_k=int(rng.choice([0, 1, 5, 40, 64, 65, 300, 5000, n])),
                      min_p=float(rng.choice([0.0, 0.05, 0.5])))
        u = rng.random(rows)
        dx = hip.array(x)
        hip.sample(dx, rows, n, u, dout, **params)
        got = dout.numpy()[:rows]
        dx.free()
        want, margin = orc.sample(x, u, **params)
        for r in range(rows):
            if got[r] != want[r]:
                assert margin[r] < 1e-6, (n, params, r, int(got[r]), int(want[r]), float(margin[r]))
            checked += 1
    dout.free()
    assert checked > 0


@pytest.mark.gpu
def test_sample_past_1024_slices(hip, orc):
    """A row of 1026 * 2048 - 3 logits: more slices (1026) than the pick kernel's 1024 threads, so the slices'
    totals go through LDS in two chunks, the walk without a filter reads the sums past the first chunk from memory,
    the threshold select reads lists past its registers and the gather from the thread summaries takes several
    rounds; each filter kind against the oracle, two rows per call (ties planted in one)."""
    n = 1026 * 2048 - 3
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((2, n)) * 3).astype(np.float32)
    x[1, rng.integers(0, n, 4)] = x[1].max()
    dx = hip.array(x)
    dout = hip.array(shape=(2,), dtype=np.int32)
    for params in (dict(temperature=0.8), dict(temperature=0.8, top_k=50), dict(temperature=0.8, top_k=3000),
                   dict(temperature=0.8, top_p=0.9), dict(temperature=1.3, min_p=0.05, top_p=0.7)):
        u = rng.random(2)
        hip.sample(dx, 2, n, u, dout, **params)
        got = dout.numpy()
        want, margin = orc.sample(x, u, **params)
        for r in range(2):
            if got[r] != want[r]:
                assert margin[r] < 1e-6, (params, r, int(got[r]), int(want[r]), float(margin[r]))
    dx.free()
    dout.free()

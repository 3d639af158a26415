"""Row kernels of the oracle (engine/src/kernels.cpp:162-234) and the Q/K producer composition
(packs/dory/dory.cpp:482-490), pinned by mathematical invariants (unit norms, RoPE as a norm-preserving rotation
that reduces to the identity at position 0, closed-form SwiGLU in FP64) and by golden vectors from the
compiled reference."""
import math
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_justnorm_unit_norm(orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, 3072)).astype(np.float32) * 3
    y = orc.justnorm(x)
    np.testing.assert_allclose(np.linalg.norm(y.astype(np.float64), axis=1), 1.0, rtol=1e-6)
    np.testing.assert_allclose(y, x / np.sqrt((x.astype(np.float64) ** 2).sum(1, keepdims=True) + 1e-6), rtol=2e-6,
                               atol=1e-9)


def test_slerp_endpoints(orc):
    """lr = 0 gives justnorm(a); lr = 1 gives justnorm(b); the result is always unit norm."""
    rng = np.random.default_rng(2)
    a = rng.standard_normal((2, 512)).astype(np.float32)
    b = rng.standard_normal((2, 512)).astype(np.float32)
    np.testing.assert_allclose(orc.slerp_residual(a, b, np.zeros(512, np.float32)), orc.justnorm(a), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(orc.slerp_residual(a, b, np.ones(512, np.float32)), orc.justnorm(b), rtol=1e-5, atol=1e-7)
    y = orc.slerp_residual(a, b, rng.uniform(0, 1, 512).astype(np.float32))
    np.testing.assert_allclose(np.linalg.norm(y.astype(np.float64), axis=1), 1.0, rtol=1e-6)


def test_rope_rotation(orc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 4, 128)).astype(np.float32)
    np.testing.assert_array_equal(orc.rope(x, 4, 128, 0, 1e6)[0], x[0])   # position 0: angle 0
    y = orc.rope(x, 4, 128, 40000, 1e6)
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)
    # NeoX pairing (i, i + 64) with angle pos * theta^(-2i/d), checked in FP64 against FP32 angles
    half = 64
    # powf is correctly rounded here: the FP64 power rounded to FP32 (the exponent 2i/128 is exact in FP32)
    inv = np.array([np.float32(1) / np.float32(math.pow(1e6, 2 * i / 128)) for i in range(half)], dtype=np.float32)
    ang = (np.float32(40001) * inv).astype(np.float32).astype(np.float64)
    x1, x2 = x[1, :, :half].astype(np.float64), x[1, :, half:].astype(np.float64)
    ref = np.concatenate([x1 * np.cos(ang) - x2 * np.sin(ang), x2 * np.cos(ang) + x1 * np.sin(ang)], axis=-1)
    np.testing.assert_allclose(y[1], ref, atol=2e-6)


def test_rope_table_matches_rope(orc):
    cs = orc.rope_table(3, 128, 40000, 1e6)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 1, 128)).astype(np.float32)
    y = orc.rope(x, 1, 128, 40000, 1e6)
    c, s = cs[:3], cs[3:]
    ref = np.concatenate([x[:, 0, :64] * c - x[:, 0, 64:] * s, x[:, 0, 64:] * c + x[:, 0, :64] * s], axis=-1)
    # the oracle (like the reference build) contracts x1 * c - x2 * s into an FMA: equal to rounding
    np.testing.assert_allclose(y[:, 0], ref.astype(np.float32), rtol=0, atol=1e-6)


def test_swiglu_closed_form(orc):
    rng = np.random.default_rng(5)
    g = rng.standard_normal((2, 256)).astype(np.float32)
    u = rng.standard_normal((2, 256)).astype(np.float32)
    sg = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    su = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    z = g.astype(np.float64) * sg
    ref = z / (1 + np.exp(-z)) * (u.astype(np.float64) * su)
    np.testing.assert_allclose(orc.swiglu_scaled(g, u, sg, su), ref, rtol=1e-5, atol=1e-6)


def test_qk_produce(orc):
    """RoPE then per-head norm then q * qscale; k normalised and not scaled."""
    rng = np.random.default_rng(6)
    q = rng.standard_normal((2, 32, 128)).astype(np.float32)
    k = rng.standard_normal((2, 8, 128)).astype(np.float32)
    qs = rng.uniform(0.5, 1.5, 32 * 128).astype(np.float32)
    qo, ko = orc.qk_produce(q, k, 32, 8, 128, 40000, 1e6, qs)
    rq = orc.justnorm(orc.rope(q, 32, 128, 40000, 1e6).reshape(-1, 128)).reshape(2, 32 * 128) * qs
    rk = orc.justnorm(orc.rope(k, 8, 128, 40000, 1e6).reshape(-1, 128)).reshape(2, 8, 128)
    np.testing.assert_array_equal(qo.reshape(2, -1), rq)
    np.testing.assert_array_equal(ko, rk)
    np.testing.assert_allclose(np.linalg.norm(ko, axis=-1), 1.0, rtol=1e-6)


def test_rows_golden(orc):
    d = np.load(os.path.join(GOLDEN, "rows.npz"))
    tol = dict(rtol=0, atol=1e-6)
    np.testing.assert_allclose(orc.justnorm(d["x"]), d["justnorm"], **tol)
    np.testing.assert_allclose(orc.slerp_residual(d["x"], d["b"], d["lr"]), d["slerp"], **tol)
    np.testing.assert_allclose(orc.rope(d["qk"], 5, 128, 40000, 1e6), d["rope"], **tol)
    np.testing.assert_allclose(orc.swiglu_scaled(d["g"], d["u"], d["sg"], d["su"]), d["swiglu"], **tol)


@pytest.mark.skipif(not __import__("oracle").ref_available(), reason="oracle/_ref not built (no reference tree)")
def test_rows_vs_reference_bitwise(orc):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((5, 3072)).astype(np.float32)
    b = rng.standard_normal((5, 3072)).astype(np.float32)
    lr = rng.uniform(0, 0.2, 3072).astype(np.float32)
    np.testing.assert_array_equal(orc.justnorm(x), orc.justnorm(x, use_ref=True))
    np.testing.assert_array_equal(orc.slerp_residual(x, b, lr), orc.slerp_residual(x, b, lr, use_ref=True))
    qk = rng.standard_normal((8, 40, 128)).astype(np.float32)
    np.testing.assert_array_equal(orc.rope(qk, 40, 128, 39999, 1e6), orc.rope(qk, 40, 128, 39999, 1e6, use_ref=True))


def argmax_cases():
    """Rows with known answers: ties go to the first index, NaNs never win, a NaN at 0 is never displaced, -inf
    everywhere gives 0."""
    nan, inf = np.float32("nan"), np.float32("inf")
    return [([1, 3, 3, 2], 1), ([5, 1, 5], 0), ([nan, 5, 6], 0), ([1, nan, 0.5], 0), ([-1, nan, 7, 7, nan], 2),
            ([-inf, -inf], 0), ([-inf, nan, -1], 2), ([0.0, -0.0], 0), ([-0.0, 0.0], 0), ([2], 0),
            ([-3, -2, -2.5, -2], 1)]


def test_argmax_known_answers(orc):
    for row, want in argmax_cases():
        assert int(orc.argmax(np.array(row, np.float32))[0]) == want, row


@pytest.mark.skipif(not __import__("oracle").ref_available(), reason="oracle/_ref not built (no reference tree)")
def test_argmax_vs_reference(orc):
    """The reference's own xtg::argmax on the known-answer rows and on 131072-wide rows with planted ties and NaNs."""
    for row, _ in argmax_cases():
        x = np.array(row, np.float32)
        assert orc.argmax(x, use_ref=True)[0] == orc.argmax(x)[0]
    rng = np.random.default_rng(7)
    x = np.round(rng.standard_normal((6, 131072)) * 4).astype(np.float32)   # many equal values
    x[1, 0] = np.nan
    x[2, ::3] = np.nan
    x[3, 5000] = x[3, 90000] = x[3].max() + 1
    np.testing.assert_array_equal(orc.argmax(x, use_ref=True), orc.argmax(x))


def test_sample_known_answers(orc):
    """xtg::Sampler::sample (sampler.cpp:40-94) where the answer is fixed by the definition: temperature 0 is
    argmax; top_k 1 and a tiny top_p keep only the most likely (ties: the smaller index); min_p 1 keeps the maxima
    and their ties in index order; equal logits without a filter are walked in index order, so the draw u picks
    index floor(u n); a single finite logit is always chosen."""
    x = np.array([0.5, 2.0, 2.0, -1.0, 1.5], np.float32)
    assert orc.sample(x[None], [0.9], temperature=0.0)[0][0] == 1
    for u in (0.0, 0.5, 0.999):
        assert orc.sample(x[None], [u], top_k=1)[0][0] == 1
        assert orc.sample(x[None], [u], top_p=1e-4)[0][0] == 1
    # min_p 1: the two maxima, index order, mass split evenly
    assert orc.sample(x[None], [0.49], min_p=1.0)[0][0] == 1
    assert orc.sample(x[None], [0.51], min_p=1.0)[0][0] == 2
    flat = np.zeros((1, 1000), np.float32)
    for u in (0.0, 0.1234, 0.5, 0.98765):
        assert orc.sample(flat, [u])[0][0] == int(u * 1000)
    one = np.full((1, 50), -np.inf, np.float32)
    one[0, 17] = 3.0
    for u in (0.0, 0.7):
        assert orc.sample(one, [u], temperature=0.8, top_p=0.9)[0][0] == 17
    # temperature: T -> 0 concentrates on the max; large T flattens towards index order
    y = np.array([[0.0, 1.0]], np.float32)
    assert orc.sample(y, [0.3], temperature=0.01)[0][0] == 1
    assert orc.sample(y, [0.3], temperature=1e6)[0][0] == 0 and orc.sample(y, [0.7], temperature=1e6)[0][0] == 1


def sample_params(rng, n):
    return dict(temperature=float(rng.choice([0.0, 0.3, 1.0, 2.0])), top_p=float(rng.choice([1.0, 0.9, 0.5, 0.05])),
                top_k=int(rng.choice([0, 1, 5, 40, n])), min_p=float(rng.choice([0.0, 0.05, 0.5])))


@pytest.mark.skipif(not __import__("oracle").ref_available(), reason="oracle/_ref not built (no reference tree)")
def test_sample_vs_reference(orc):
    """The reference's own Sampler, seeded, against the oracle given the draw that Sampler made: every filter
    combination, rows of 1 .. 5000 logits (past the reference's 1024-candidate sorted head) with planted ties, and
    two 131072-wide rows."""
    rng = np.random.default_rng(0)
    for trial in range(300):
        n = int(rng.choice([1, 7, 100, 1000, 5000]))
        x = (rng.standard_normal(n) * rng.choice([0.5, 2, 8])).astype(np.float32)
        if trial % 7 == 0:
            x[rng.integers(0, n, 3)] = x.max()
        params = sample_params(rng, n)
        tr, u = orc.sample_ref(x, int(rng.integers(0, 2**63)), **params)
        assert orc.sample(x[None], [u], **params)[0][0] == tr, (n, params)
    for params in (dict(temperature=1.0), dict(temperature=0.7, top_p=0.95), dict(temperature=1.0, top_k=50)):
        x = (rng.standard_normal(131072) * 3).astype(np.float32)
        tr, u = orc.sample_ref(x, 12345, **params)
        assert orc.sample(x[None], [u], **params)[0][0] == tr, params

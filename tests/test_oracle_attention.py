"""The oracle's KvCache + attention (engine/src/kv.cpp:75-286) and the ring mask by slot positions
(npu/xtg_npu.cpp:236-258), pinned by:
- a naive FP64 softmax over exactly what the cache returns (tests/kernels_test.cpp:103-183, < 2e-5 absolute),
  on the reference test's seven cases (cached / n_q / window / dtype);
- the FP8 ring keeping the last 64 of 3000 positions (tests/kernels_test.cpp:184-193);
- a planted mistake (the causal bound off by one) that the naive check must catch;
- brute-force equality of the slot-mask form and the position form on consistent rings;
- the compiled reference (oracle/_ref) and the committed golden vectors.
"""
import glob
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KT_CASES = [(300, 1, 0, 0), (5000, 1, 0, 0), (300, 1, 64, 0), (100, 37, 0, 0), (100, 37, 16, 1), (0, 20, 0, 1),
            (900, 3, 128, 1)]


def naive_attention(q, Kc, Vc, pos0, heads, kvh, d, window, scale, causal_slip=0):
    """tests/kernels_test.cpp:104-130 in FP64: positions lo(t) .. t of the explicit K / V rows."""
    n_q = q.shape[0]
    g = heads // kvh
    out = np.zeros((n_q, heads, d), dtype=np.float64)
    for i in range(n_q):
        t = pos0 + i
        lo = max(0, t - window + 1) if window > 0 else 0
        hi = t + 1 + causal_slip
        for h in range(heads):
            kh = h // g
            s = Kc[lo:hi, kh, :].astype(np.float64) @ q[i, h].astype(np.float64) * scale
            p = np.exp(s - s.max())
            out[i, h] = (p / p.sum()) @ Vc[lo:hi, kh, :].astype(np.float64)
    return out


def build_case(orc, cached, n_q, window, fp8, rng, heads=8, kvh=2, d=64, use_ref=False):
    total = cached + n_q
    K = rng.uniform(-1, 1, (total, kvh, d)).astype(np.float32)
    V = rng.uniform(-1, 1, (total, kvh, d)).astype(np.float32)
    q = rng.uniform(-1, 1, (n_q, heads, d)).astype(np.float32)
    cache = orc.KvCache(kvh, d, total + 8, ring=window if window > 0 else 0, fp8=bool(fp8), use_ref=use_ref)
    for p in range(0, cached, 50):
        n = min(50, cached - p)
        cache.store(p, K[p:p + n], V[p:p + n])
    Kc, Vc = K.copy(), V.copy()
    lo = max(0, cached - window) if window > 0 else 0
    for h in range(kvh):
        if cached > lo:
            kk, vv = cache.load(h, lo, cached)
            Kc[lo:cached, h] = kk
            Vc[lo:cached, h] = vv
    return K, V, q, cache, Kc, Vc


@pytest.mark.parametrize("cached,n_q,window,fp8", KT_CASES)
def test_attention_vs_naive(orc, cached, n_q, window, fp8):
    rng = np.random.default_rng(42)
    K, V, q, cache, Kc, Vc = build_case(orc, cached, n_q, window, fp8, rng)
    out = orc.attention(q, K[cached:], V[cached:], cache, cached, 8, 2, 64, window=window, scale=0.7, pool_size=4)
    ref = naive_attention(q, Kc, Vc, cached, 8, 2, 64, window, 0.7)
    assert np.max(np.abs(out - ref)) < 2e-5


@pytest.mark.parametrize("cached,n_q,window,fp8", [(300, 1, 0, 0), (200, 9, 0, 1), (500, 3, 64, 1)])
def test_attention_head_dim_256(orc, cached, n_q, window, fp8):
    """The real Dory 4B's heads (16 q over 4 KV heads of 256, docs/dory.md:13): FP64 and the compiled reference."""
    rng = np.random.default_rng(256)
    K, V, q, cache, Kc, Vc = build_case(orc, cached, n_q, window, fp8, rng, heads=16, kvh=4, d=256)
    out = orc.attention(q, K[cached:], V[cached:], cache, cached, 16, 4, 256, window=window, scale=0.7, pool_size=4)
    assert np.max(np.abs(out - naive_attention(q, Kc, Vc, cached, 16, 4, 256, window, 0.7))) < 2e-5
    if orc.ref_available():
        rng = np.random.default_rng(256)
        K2, V2, q2, cache_r, _, _ = build_case(orc, cached, n_q, window, fp8, rng, heads=16, kvh=4, d=256, use_ref=True)
        ref = orc.attention(q2, K2[cached:], V2[cached:], cache_r, cached, 16, 4, 256, window=window, scale=0.7,
                            pool_size=4)
        assert np.max(np.abs(out - ref)) <= 1e-6


def test_naive_catches_causal_slip(orc):
    rng = np.random.default_rng(43)
    K, V, q, cache, Kc, Vc = build_case(orc, 100, 37, 0, 0, rng)
    out = orc.attention(q, K[100:], V[100:], cache, 100, 8, 2, 64, scale=0.7, pool_size=4)
    wrong = naive_attention(q, Kc, Vc, 100, 8, 2, 64, 0, 0.7, causal_slip=1)
    assert np.max(np.abs(out - wrong)) > 1e-3


def test_fp8_ring_keeps_last_positions(orc):
    """tests/kernels_test.cpp:184-193."""
    rng = np.random.default_rng(44)
    ring = orc.KvCache(1, 64, 0, ring=64, fp8=True)
    k = rng.uniform(-0.3, 0.3, (3000, 1, 64)).astype(np.float32)
    v = rng.uniform(-2, 2, (3000, 1, 64)).astype(np.float32)
    ring.store(0, k, v)
    kb, vb = ring.load(0, 2936, 3000)
    assert np.max(np.abs(kb - k[2936:, 0])) / 0.3 < 0.07


@pytest.mark.parametrize("window,slots,n_q", [(16, 24, 1), (16, 24, 5), (64, 80, 8), (1024, 1088, 8), (1088, 1088, 8)])
def test_slot_mask_equals_position_form(orc, window, slots, n_q):
    """With a ring written in position order, the slot-position mask of the NPU plugin and the CPU kernel's
    position window select the same keys; the outputs agree to FP32 rounding."""
    rng = np.random.default_rng(window + slots + n_q)
    heads, kvh, d = 8, 2, 32
    pos0 = 3 * slots + 11
    cache = orc.KvCache(kvh, d, 0, ring=slots)
    K = rng.uniform(-1, 1, (pos0 + n_q, kvh, d)).astype(np.float32)
    V = rng.uniform(-1, 1, (pos0 + n_q, kvh, d)).astype(np.float32)
    for p in range(0, pos0, 37):
        n = min(37, pos0 - p)
        cache.store(p, K[p:p + n], V[p:p + n])
    slot_pos = np.full(slots, -1, dtype=np.int64)
    for p in range(pos0):
        slot_pos[p % slots] = p
    q = rng.uniform(-1, 1, (n_q, heads, d)).astype(np.float32)
    by_pos = orc.attention(q, K[pos0:], V[pos0:], cache, pos0, heads, kvh, d, window=window, pool_size=1)
    by_slot = orc.attention(q, K[pos0:], V[pos0:], cache, pos0, heads, kvh, d, window=window, slot_pos=slot_pos)
    assert np.max(np.abs(by_pos - by_slot)) < 2e-6


def test_slot_mask_hides_unwritten_and_stale_slots(orc):
    """Slots with position -1 (never written) or outside the window are not attended: the result equals the
    attention over the visible slots only, computed naively."""
    rng = np.random.default_rng(9)
    heads, kvh, d, slots, window = 4, 1, 16, 32, 20
    cache = orc.KvCache(kvh, d, 0, ring=slots)
    pos0 = 25   # the ring has seen positions 0..24: slots 25..31 unwritten
    K = rng.uniform(-1, 1, (pos0 + 2, kvh, d)).astype(np.float32)
    V = rng.uniform(-1, 1, (pos0 + 2, kvh, d)).astype(np.float32)
    cache.store(0, K[:pos0], V[:pos0])
    slot_pos = np.array([p if p < pos0 else -1 for p in range(slots)], dtype=np.int64)
    q = rng.uniform(-1, 1, (2, heads, d)).astype(np.float32)
    out = orc.attention(q, K[pos0:], V[pos0:], cache, pos0, heads, kvh, d, window=window, slot_pos=slot_pos)
    Kc = wl_round(K)
    Vc = wl_round(V)
    Kc[pos0:], Vc[pos0:] = K[pos0:], V[pos0:]
    ref = naive_attention(q, Kc, Vc, pos0, heads, kvh, d, window, float(np.float32(1) / np.sqrt(np.float32(d))))
    assert np.max(np.abs(out - ref)) < 2e-5


def wl_round(a):
    """BF16 round trip of an FP32 array (what a BF16 cache returns)."""
    b = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = ((b + np.uint32(0x7FFF) + ((b >> 16) & 1)) >> 16).astype(np.uint32) << 16
    return r.view(np.float32).reshape(a.shape)


@pytest.mark.skipif(not __import__("oracle").ref_available(), reason="oracle/_ref not built (no reference tree)")
@pytest.mark.parametrize("cached,n_q,window,fp8", KT_CASES[:4] + [(2000, 8, 0, 0), (3000, 1, 1024, 0)])
def test_attention_vs_reference(orc, cached, n_q, window, fp8):
    rng = np.random.default_rng(7)
    K, V, q, cache, _, _ = build_case(orc, cached, n_q, window, fp8, rng)
    rng = np.random.default_rng(7)
    K2, V2, q2, cache_r, _, _ = build_case(orc, cached, n_q, window, fp8, rng, use_ref=True)
    for pool in (1, 4, 16):
        mine = orc.attention(q, K[cached:], V[cached:], cache, cached, 8, 2, 64, window=window, scale=0.7, pool_size=pool)
        ref = orc.attention(q2, K2[cached:], V2[cached:], cache_r, cached, 8, 2, 64, window=window, scale=0.7,
                            pool_size=pool)
        assert np.max(np.abs(mine - ref)) <= 1e-6


def test_attention_golden(orc):
    files = sorted(glob.glob(os.path.join(GOLDEN, "attn_*.npz")))
    assert files, "no golden attention vectors committed"
    for f in files:
        d = np.load(f)
        cached, window, fp8 = int(d["cached"]), int(d["window"]), int(d["fp8"])
        heads, kvh, hd = int(d["heads"]), int(d["kv_heads"]), int(d["head_dim"])
        q = d["q"]
        n_q = q.shape[0]
        if fp8:
            K, V = d["K"], d["V"]
        else:
            K = np.concatenate([(d["Kc"].astype(np.uint32) << 16).view(np.float32), d["Kn"]])
            V = np.concatenate([(d["Vc"].astype(np.uint32) << 16).view(np.float32), d["Vn"]])
        cache = orc.KvCache(kvh, hd, cached + n_q + 8, ring=window if window > 0 else 0, fp8=bool(fp8))
        for p in range(0, cached, 50):
            n = min(50, cached - p)
            cache.store(p, K[p:p + n], V[p:p + n])
        out = orc.attention(q, K[cached:], V[cached:], cache, cached, heads, kvh, hd, window=window,
                            scale=float(d["scale"]), pool_size=int(d["pool_size"]))
        assert np.max(np.abs(out - d["out"])) <= 1e-6, f

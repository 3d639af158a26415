"""GPU parity of the device KV cache (xtg_hip_kv_*) and decode attention (xtg_hip_attention) against the oracle's
KvCache + attention (engine/src/kv.cpp:75-286) and ring mask (npu/xtg_npu.cpp:236-258), on the same seeded inputs.

Bars: KV store / load bit-exact (BF16 round to nearest even; FP8 codes and per-(position, head) scales as
kv.cpp:19-40, 94-108 make them); attention rel-L2 <= 1e-5 against the oracle and max |err| <= 2e-5 against an FP64
softmax of exactly what the cache holds (tests/kernels_test.cpp:103-183's bar); for the sharp cases (scores up to
~20) rel-L2 <= 5e-5 against the oracle, whose own FP32 error is of that order.
"""
import glob
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def rel_l2(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(np.asarray(y, np.float64) - ref) / np.linalg.norm(ref))


def bf16_round(a):
    b = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = ((b + np.uint32(0x7FFF) + ((b >> 16) & 1)) >> 16).astype(np.uint32) << 16
    return r.view(np.float32).reshape(np.shape(a))


def naive(q, Kc, Vc, pos0, heads, kvh, window, scale):
    """FP64 softmax attention over explicit rows Kc / Vc [positions][kvh][d] (tests/kernels_test.cpp:104-130)."""
    n_q, d = q.shape[0], q.shape[2]
    g = heads // kvh
    out = np.zeros((n_q, heads, d))
    for i in range(n_q):
        t = pos0 + i
        lo = max(0, t - window + 1) if window > 0 else 0
        for h in range(heads):
            s = Kc[lo:t + 1, h // g].astype(np.float64) @ q[i, h].astype(np.float64) * scale
            p = np.exp(s - s.max())
            out[i, h] = (p / p.sum()) @ Vc[lo:t + 1, h // g].astype(np.float64)
    return out


def run_case(hip, orc, cached, n_q, window, heads, kvh, d, scale, rng, ring=None, qmul=1.0, unit=False, fp8=False):
    total = cached + n_q
    if unit:
        K = rng.standard_normal((total, kvh, d)).astype(np.float32)
        K /= np.linalg.norm(K, axis=-1, keepdims=True)
        V = rng.standard_normal((total, kvh, d)).astype(np.float32)
        V /= np.linalg.norm(V, axis=-1, keepdims=True)
        q = rng.standard_normal((n_q, heads, d)).astype(np.float32)
        q /= np.linalg.norm(q, axis=-1, keepdims=True)
    else:
        K = rng.uniform(-1, 1, (total, kvh, d)).astype(np.float32)
        V = rng.uniform(-1, 1, (total, kvh, d)).astype(np.float32)
        q = rng.uniform(-1, 1, (n_q, heads, d)).astype(np.float32)
    q = (q * np.float32(qmul)).astype(np.float32)
    ring = ring if ring is not None else (window if window > 0 else 0)
    oc = orc.KvCache(kvh, d, total + 8, ring=ring, fp8=fp8)
    dc = hip.kv_cache(kvh, d, total + 8, ring=ring, dtype=1 if fp8 else 0)
    for p in range(0, cached, 50):
        n = min(50, cached - p)
        oc.store(p, K[p:p + n], V[p:p + n])
        dc.store_host(p, K[p:p + n], V[p:p + n])
    ref = orc.attention(q, K[cached:], V[cached:], oc, cached, heads, kvh, d, window=window, scale=scale, pool_size=4)
    dq, dk, dv = hip.array(q), hip.array(K[cached:]), hip.array(V[cached:])
    dout = hip.array(shape=q.shape)
    hip.attention(dc, dq, dk, dv, dout, n_q, cached, heads, window=window, scale=scale)
    out = dout.numpy()
    for a in (dq, dk, dv, dout):
        a.free()
    exact = None
    if cached * n_q <= 400000:   # FP64 softmax over what the cache holds (the oracle's load) and the FP32 own rows
        Kc, Vc = K.copy(), V.copy()
        lo = max(0, cached - ring) if ring > 0 else 0
        for h in range(kvh):
            if cached > lo:
                Kc[lo:cached, h], Vc[lo:cached, h] = oc.load(h, lo, cached)
        sc = scale if scale is not None else float(np.float32(1) / np.sqrt(np.float32(d)))
        exact = naive(q, Kc, Vc, cached, heads, kvh, window, sc)
    dc.destroy()
    return out, ref, exact


# tests/kernels_test.cpp:139-141: (cached, n_q, window, FP8 cache)
KT = [(300, 1, 0, 0), (5000, 1, 0, 0), (300, 1, 64, 0), (100, 37, 0, 0), (100, 37, 16, 1), (0, 20, 0, 1),
      (900, 3, 128, 1)]


@pytest.mark.parametrize("cached,n_q,window,fp8", KT)
def test_reference_unit_cases(hip, orc, cached, n_q, window, fp8):
    rng = np.random.default_rng(42 + cached + n_q + window)
    out, ref, exact = run_case(hip, orc, cached, n_q, window, 8, 2, 64, 0.7, rng, fp8=bool(fp8))
    assert rel_l2(out, ref) <= 1e-5
    if exact is not None:
        assert np.max(np.abs(out - exact)) < 2e-5


@pytest.mark.parametrize("cached,n_q,window,fp8", [(1500, 300, 0, 0), (1500, 300, 256, 1), (0, 129, 0, 0),
                                                   (2000, 512, 1024, 0)])
def test_prefill_rows(hip, orc, cached, n_q, window, fp8):
    """Prefill-sized calls (many row blocks, the last one partial, in one own-key and one scan launch) on the
    4B model's heads: 32 query heads over 8 KV heads of 128."""
    rng = np.random.default_rng(cached + n_q + window + fp8)
    out, ref, _ = run_case(hip, orc, cached, n_q, window, 32, 8, 128, None, rng, unit=True, fp8=bool(fp8))
    assert rel_l2(out, ref) <= 1e-5


@pytest.mark.parametrize("ctx", [4096, 8192, 32768])
@pytest.mark.parametrize("n_q", [1, 8])
def test_decode_global_cache(hip, orc, ctx, n_q):
    """Global-cache decode attention: 32 q / 8 KV heads of 128, unit-norm K / V / q, BF16 cache of ctx positions,
    1 or 8 new rows."""
    rng = np.random.default_rng(ctx + n_q)
    out, ref, _ = run_case(hip, orc, ctx, n_q, 0, 32, 8, 128, None, rng, unit=True)
    assert rel_l2(out, ref) <= 1e-5


@pytest.mark.parametrize("ctx,n_q", [(4096, 1), (4096, 8), (32768, 1), (32768, 8)])
def test_decode_global_cache_fp8(hip, orc, ctx, n_q):
    """The global-cache shapes over an FP8 cache (the reference Dory's default KV dtype, dory.cpp:141)."""
    rng = np.random.default_rng(ctx + n_q + 1)
    out, ref, _ = run_case(hip, orc, ctx, n_q, 0, 32, 8, 128, None, rng, unit=True, fp8=True)
    assert rel_l2(out, ref) <= 1e-5


# Calls of one row block with cached keys take their own keys and the scan in one launch and the merge by heads;
# XTG_ATTN_UNFUSED=1 takes the own-key, scan and merge launches. (heads, kv_heads, d, cached, n_q, window, fp8)
ONE_BLOCK = [(32, 8, 128, 4096, 1, 0, 0), (32, 8, 128, 4096, 8, 0, 1), (32, 8, 128, 3000, 5, 1024, 0),
             (16, 4, 256, 700, 5, 64, 1), (8, 2, 64, 500, 3, 0, 0), (16, 2, 128, 700, 4, 0, 1),
             (32, 8, 128, 0, 8, 0, 0)]


@pytest.mark.parametrize("heads,kvh,d,cached,n_q,window,fp8", ONE_BLOCK)
def test_one_block_call_fused_and_three_launches(hip, orc, monkeypatch, heads, kvh, d, cached, n_q, window, fp8):
    """The same call both ways on the same inputs: the launches name the path taken (one launch for the own keys
    and the scan, then attn_merge_heads_kernel; with nothing cached the three launches either way), the two outputs
    agree within 2e-6 and each is within the oracle bar of 1e-5."""
    outs = []
    for unfused in (False, True):
        if unfused:
            monkeypatch.setenv("XTG_ATTN_UNFUSED", "1")
        rng = np.random.default_rng(900 + heads + d + cached + n_q + window + fp8)
        hip.profile(True, launches=True)
        out, ref, _ = run_case(hip, orc, cached, n_q, window, heads, kvh, d, None, rng, unit=True, fp8=bool(fp8))
        _, launches = hip.profile_report(launches=True)
        hip.profile(False)
        names = [n for n, _ in launches]
        fused = any(n.startswith("attn_step_kernel") for n in names)
        assert fused == (cached > 0 and not unfused), names
        assert any(n.startswith("attn_merge_heads_kernel") for n in names) == fused, names
        assert rel_l2(out, ref) <= 1e-5
        outs.append(out)
    monkeypatch.delenv("XTG_ATTN_UNFUSED")
    assert rel_l2(outs[0], outs[1]) <= 2e-6


# The real Dory 4B's attention (docs/dory.md:13): 16 q heads over 4 KV heads of 256. (cached, n_q, window, FP8):
# decode and verify steps over global caches, a prefill chunk, sliding windows over rings of window + 16 slots
# (the CPU session's ring, packs/dory/dory.cpp:43, 449), a call with nothing cached.
D256 = [(4096, 1, 0, 0), (4096, 8, 0, 0), (4096, 1, 0, 1), (8192, 8, 0, 1), (300, 37, 0, 0), (1500, 300, 0, 1),
        (3000, 8, 1024, 1), (3000, 1, 1024, 0), (0, 20, 0, 0), (700, 5, 64, 1)]


@pytest.mark.parametrize("cached,n_q,window,fp8", D256)
def test_head_dim_256(hip, orc, cached, n_q, window, fp8):
    rng = np.random.default_rng(256 + cached + n_q + window + fp8)
    out, ref, exact = run_case(hip, orc, cached, n_q, window, 16, 4, 256, None, rng, unit=True, fp8=bool(fp8),
                               ring=window + 16 if window else 0)
    assert rel_l2(out, ref) <= 1e-5
    if exact is not None:
        assert np.max(np.abs(out - exact)) < 2e-5


@pytest.mark.parametrize("n_q", [1, 8])
def test_head_dim_256_sharp(hip, orc, n_q):
    """A sharp softmax (q x 30) at 256 dims over an FP8 cache of 900 keys."""
    rng = np.random.default_rng(2560 + n_q)
    out, ref, exact = run_case(hip, orc, 900, n_q, 0, 16, 4, 256, None, rng, unit=True, qmul=30.0, fp8=True)
    assert rel_l2(out, ref) <= 5e-5
    assert rel_l2(out, exact) <= max(3 * rel_l2(ref, exact), 1e-5)


@pytest.mark.parametrize("n_q", [1, 5, 16])
def test_head_dim_128_group_8_fp8(hip, orc, n_q):
    """Eight q heads per KV head (two q-blocks per MFMA pass at 4+ rows), FP8, a sharp softmax, 700 cached keys."""
    rng = np.random.default_rng(70 + n_q)
    out, ref, exact = run_case(hip, orc, 700, n_q, 0, 16, 2, 128, None, rng, unit=True, qmul=30.0, fp8=True)
    assert rel_l2(out, ref) <= 5e-5
    assert rel_l2(out, exact) <= max(3 * rel_l2(ref, exact), 1e-5)


def test_golden_vectors(hip):
    """The committed golden vectors (the seven unit cases and the 320-position configs, made by the oracle and
    checked against the compiled reference) through the device cache and attention."""
    files = sorted(glob.glob(os.path.join(GOLDEN, "attn_*.npz")))
    assert files
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
        dc = hip.kv_cache(kvh, hd, cached + n_q + 8, ring=window if window > 0 else 0, dtype=fp8)
        for p in range(0, cached, 50):
            n = min(50, cached - p)
            dc.store_host(p, K[p:p + n], V[p:p + n])
        dq, dk, dv = hip.array(q), hip.array(np.ascontiguousarray(K[cached:])), hip.array(np.ascontiguousarray(V[cached:]))
        dout = hip.array(shape=q.shape)
        hip.attention(dc, dq, dk, dv, dout, n_q, cached, heads, window=window, scale=float(d["scale"]))
        out = dout.numpy()
        for a in (dq, dk, dv, dout):
            a.free()
        dc.destroy()
        assert rel_l2(out, d["out"]) <= 1e-5, f


@pytest.mark.parametrize("qmul", [60.0, 250.0])
def test_decode_sharp_softmax(hip, orc, qmul):
    """Peaked softmax (q scaled so that scores reach tens): the three-term q split keeps FP32-level scores."""
    rng = np.random.default_rng(int(qmul))
    out, ref, exact = run_case(hip, orc, 600, 8, 0, 32, 8, 128, None, rng, unit=True, qmul=qmul)
    assert rel_l2(out, ref) <= 5e-5
    err_gpu = rel_l2(out, exact)
    err_cpu = rel_l2(ref, exact)
    assert err_gpu <= max(3 * err_cpu, 1e-5), (err_gpu, err_cpu)


@pytest.mark.parametrize("qmul,n_q,fp8", [(200.0, 1, False), (200.0, 8, False), (2000.0, 1, False),
                                           (2000.0, 8, False), (2000.0, 1, True), (2000.0, 8, True)])
def test_decode_sharp_softmax_32k(hip, orc, qmul, n_q, fp8):
    """The 4B model's global cache at 32768 positions (the plan's 24 key splits, 64 for one row of an FP8 cache,
    merged across splits) under a peaked softmax: unit q scaled by 200 (scores of std ~1.6 over the keys) and by 2000
    (std ~16: the largest scores ~70, a few keys carry the weight, as Dory's scores in the hundreds do); BF16 and FP8
    caches, 1 and 8 rows. Against the oracle at 5e-5 and against an FP64 softmax of what the cache holds at 3x the
    oracle's own error."""
    rng = np.random.default_rng(int(qmul) + n_q + 7 * fp8)
    out, ref, exact = run_case(hip, orc, 32768, n_q, 0, 32, 8, 128, None, rng, unit=True, qmul=qmul, fp8=fp8)
    assert exact is not None
    assert rel_l2(out, ref) <= 5e-5
    err_gpu, err_cpu = rel_l2(out, exact), rel_l2(ref, exact)
    assert err_gpu <= max(3 * err_cpu, 1e-5), (err_gpu, err_cpu)


@pytest.mark.parametrize("window,fp8", [(1024, False), (1088, False), (1024, True)])
def test_ring_wrapped_1088_slots(hip, orc, wl, window, fp8):
    """The sliding-window ring: a 1088-slot ring after 40000 positions (holding 38912..39999), 8 rows at
    40000..40007, q and k produced by RoPE (theta 1e6) -> per-head norm -> q * qscale ~ U(0.5, 1.5); the mask is rebuilt from the stored
    slot positions. Compared with the oracle's position form and its slot form."""
    rng = np.random.default_rng(window)
    heads, kvh, d, ring, pos0, n_q = 32, 8, 128, 1088, 40000, 8
    Kr = wl.unit_heads(rng, (ring, kvh), d)
    Vr = wl.unit_heads(rng, (ring, kvh), d)
    first = pos0 - ring
    oc = orc.KvCache(kvh, d, 0, ring=ring, fp8=fp8)
    dc = hip.kv_cache(kvh, d, 0, ring=ring, dtype=1 if fp8 else 0)
    oc.store(first, Kr, Vr)
    dc.store_host(first, Kr, Vr)
    slot_pos = np.full(ring, -1, np.int64)
    for p in range(first, pos0):
        slot_pos[p % ring] = p
    q = rng.standard_normal((n_q, heads, d)).astype(np.float32)
    k = rng.standard_normal((n_q, kvh, d)).astype(np.float32)
    v = wl.unit_heads(rng, (n_q, kvh), d)
    qscale = rng.uniform(0.5, 1.5, heads * d).astype(np.float32)
    qo, ko = orc.qk_produce(q, k, heads, kvh, d, pos0, 1e6, qscale)
    ref = orc.attention(qo, ko, v, oc, pos0, heads, kvh, d, window=window, pool_size=4)
    ref_slots = orc.attention(qo, ko, v, oc, pos0, heads, kvh, d, window=window, slot_pos=slot_pos)
    dq, dk, dv = hip.array(q), hip.array(k), hip.array(v)
    dqs = hip.array(qscale)
    dout = hip.array(shape=(n_q, heads, d))
    hip.qk_rope_norm(dq, dk, n_q, heads, kvh, d, pos0, 1e6, dqs)
    hip.attention(dc, dq, dk, dv, dout, n_q, pos0, heads, window=window)
    out = dout.numpy()
    qg, kg = dq.numpy(), dk.numpy()
    for a in (dq, dk, dv, dqs, dout):
        a.free()
    dc.destroy()
    assert rel_l2(qg, qo) <= 1e-6 and rel_l2(kg, ko) <= 1e-6
    assert rel_l2(out, ref) <= 1e-5
    assert rel_l2(out, ref_slots) <= 1e-5


def test_kv_store_load_roundtrip(hip, orc):
    """Store in chunks (linear and ring), load back: the BF16 bits the oracle's cache returns, exactly."""
    rng = np.random.default_rng(5)
    kvh, d = 8, 128
    K = rng.standard_normal((700, kvh, d)).astype(np.float32)
    V = rng.standard_normal((700, kvh, d)).astype(np.float32)
    for ring in (0, 96):
        oc = orc.KvCache(kvh, d, 800, ring=ring)
        dc = hip.kv_cache(kvh, d, 800, ring=ring)
        for p in range(0, 700, 70):
            oc.store(p, K[p:p + 70], V[p:p + 70])
            dc.store_host(p, K[p:p + 70], V[p:p + 70])
        lo = 700 - 96 if ring else 0
        for h in (0, 3, 7):
            ok, ov = oc.load(h, lo, 700)
            gk, gv = dc.load(h, lo, 700)
            np.testing.assert_array_equal(gk, ok)
            np.testing.assert_array_equal(gv, ov)
        dc.destroy()


def fp8_rows(rng, n, kvh, d):
    """Random rows plus rows that hit the E4M3 rounding's edges: amax 448 (scale 1) with values at ties between
    codes (normal and subnormal), below the smallest subnormal step, an all-zero row (scale 1), a row of one
    nonzero, negative zero, and a NaN (its code 0x7f; the scale ignores it)."""
    K = rng.standard_normal((n, kvh, d)).astype(np.float32)
    ties = np.array([448.0, 1.0625, 1.1875, -1.0625, 3 * 2.0 ** -10, 5 * 2.0 ** -10, 2.0 ** -11, 2.0 ** -12,
                     0.0, -0.0, 2.0 ** -6 - 2.0 ** -11, 15.5 * 2.0 ** -10, 240.0, 232.0, 0.5 + 2.0 ** -5,
                     300.0], np.float32)
    K[0, 0, :ties.size] = ties
    K[0, 0, ties.size:] = 0.25
    K[1, 0] = 0.0
    K[2, 0] = 0.0
    K[2, 0, 5] = -3e-5
    K[3, 0, 7] = np.nan
    return K


def test_kv_fp8_store_load_bits(hip, orc):
    """FP8 rows stored in chunks (linear and ring) and by one long call: the loaded values (code value x scale)
    equal the oracle's bit for bit, and so do the per-(position, head) scales in the device snapshot."""
    rng = np.random.default_rng(15)
    kvh, d, n = 4, 128, 300
    K = fp8_rows(rng, n, kvh, d)
    V = fp8_rows(rng, n, kvh, d)[::-1].copy()
    for ring, chunk in ((0, 37), (96, 37), (0, n)):
        oc = orc.KvCache(kvh, d, 320, ring=ring, fp8=True)
        dc = hip.kv_cache(kvh, d, 320, ring=ring, dtype=1)
        for p in range(0, n, chunk):
            oc.store(p, K[p:p + chunk], V[p:p + chunk])
            dc.store_host(p, K[p:p + chunk], V[p:p + chunk])
        lo = n - ring if ring else 0
        for h in range(kvh):
            ok, ov = oc.load(h, lo, n)
            gk, gv = dc.load(h, lo, n)
            np.testing.assert_array_equal(gk.view(np.uint32), ok.view(np.uint32))
            np.testing.assert_array_equal(gv.view(np.uint32), ov.view(np.uint32))
        # snapshot: K codes, V codes, K scales [head][slot], V scales, slot positions
        snap = dc.save()
        slots = ring if ring else 320
        pad = (slots + 31) // 32 * 32
        data = kvh * pad * d
        ks = snap[2 * data:2 * data + 4 * kvh * pad].view(np.float32).reshape(kvh, pad)
        vs = snap[2 * data + 4 * kvh * pad:2 * data + 8 * kvh * pad].view(np.float32).reshape(kvh, pad)
        oks, ovs = oc.scales()
        for p in range(lo, n):
            s = p % slots if ring else p
            np.testing.assert_array_equal(ks[:, s], oks[s])
            np.testing.assert_array_equal(vs[:, s], ovs[s])
        dc.destroy()


def test_kv_fp8_save_restore(hip, orc):
    rng = np.random.default_rng(16)
    kvh, d = 2, 64
    K = rng.standard_normal((64, kvh, d)).astype(np.float32)
    V = rng.standard_normal((64, kvh, d)).astype(np.float32)
    dc = hip.kv_cache(kvh, d, 0, ring=40, dtype=1)
    oc = orc.KvCache(kvh, d, 0, ring=40, fp8=True)
    dc.store_host(0, K[:40], V[:40])
    oc.store(0, K[:40], V[:40])
    snap = dc.save()
    assert snap.nbytes == 2 * kvh * 64 * d + 2 * 4 * kvh * 64 + 4 * 64
    dc.store_host(40, K[40:], V[40:])
    dc.restore(snap)
    for h in range(kvh):
        gk, gv = dc.load(h, 0, 40)
        ok, ov = oc.load(h, 0, 40)
        np.testing.assert_array_equal(gk, ok)
        np.testing.assert_array_equal(gv, ov)
    dc.release()
    q = rng.standard_normal((1, 4, d)).astype(np.float32)
    dq, dk, dv = hip.array(q), hip.array(K[:1]), hip.array(V[:1])
    dout = hip.array(shape=(1, 4, d))
    hip.attention(dc, dq, dk, dv, dout, 1, 40, 4)   # released: only the call's own key is visible
    out = dout.numpy()
    np.testing.assert_allclose(out[0], np.repeat(V[:1, :, :], 2, axis=1)[0], rtol=0, atol=1e-6)
    for a in (dq, dk, dv, dout):
        a.free()
    dc.destroy()


def test_kv_ring_long_store_keeps_last(hip, orc):
    """A store longer than the ring keeps its last `slots` rows (engine/src/kv.cpp:75-80)."""
    rng = np.random.default_rng(6)
    K = rng.standard_normal((300, 2, 64)).astype(np.float32)
    V = rng.standard_normal((300, 2, 64)).astype(np.float32)
    dc = hip.kv_cache(2, 64, 0, ring=64)
    dc.store_host(0, K, V)
    gk, gv = dc.load(1, 236, 300)
    np.testing.assert_array_equal(gk, bf16_round(K[236:, 1]))
    np.testing.assert_array_equal(gv, bf16_round(V[236:, 1]))
    dc.destroy()


def test_kv_save_restore_release(hip, orc):
    rng = np.random.default_rng(7)
    kvh, d = 2, 64
    K = rng.standard_normal((64, kvh, d)).astype(np.float32)
    V = rng.standard_normal((64, kvh, d)).astype(np.float32)
    dc = hip.kv_cache(kvh, d, 0, ring=40)
    dc.store_host(0, K[:40], V[:40])
    snap = dc.save()
    dc.store_host(40, K[40:], V[40:])
    dc.restore(snap)
    gk, _ = dc.load(0, 0, 40)
    np.testing.assert_array_equal(gk, bf16_round(K[:40, 0]))
    dc.release()
    q = rng.standard_normal((1, 4, d)).astype(np.float32)
    dq, dk, dv = hip.array(q), hip.array(K[:1]), hip.array(V[:1])
    dout = hip.array(shape=(1, 4, d))
    hip.attention(dc, dq, dk, dv, dout, 1, 40, 4)   # released: only the call's own key is visible
    out = dout.numpy()
    np.testing.assert_allclose(out[0], np.repeat(V[:1, :, :], 2, axis=1)[0], rtol=0, atol=1e-6)
    for a in (dq, dk, dv, dout):
        a.free()
    dc.destroy()


def test_errors(hip, pkg):
    with pytest.raises(pkg.XtgError, match="KV cache full"):
        dc = hip.kv_cache(2, 64, 32)
        try:
            dc.store_host(30, np.zeros((4, 2, 64), np.float32), np.zeros((4, 2, 64), np.float32))
        finally:
            dc.destroy()
    with pytest.raises(pkg.XtgError, match="head_dim"):
        hip.kv_cache(2, 96, 32)
    with pytest.raises(pkg.XtgError, match="head_dim"):
        hip.kv_cache(2, 512, 32)


@pytest.mark.parametrize("dtype", [0, 1])
def test_kv_copy_device_snapshot(hip, pkg, dtype):
    """A device copy (the resident session's ring snapshots) holds exactly the source's state: its host blob equals
    the source's, later stores into the source leave it unchanged, and copying it back restores the source.
    Caches of another shape are refused."""
    rng = np.random.default_rng(17 + dtype)
    kvh, d = 2, 128
    K = rng.standard_normal((150, kvh, d)).astype(np.float32)
    V = rng.standard_normal((150, kvh, d)).astype(np.float32)
    src = hip.kv_cache(kvh, d, 0, ring=96, dtype=dtype)
    snap = hip.kv_cache(kvh, d, 0, ring=96, dtype=dtype)
    other = hip.kv_cache(kvh, d, 0, ring=64, dtype=dtype)
    try:
        src.store_host(0, K[:100], V[:100])
        before = src.save()
        src.copy_to(snap)
        np.testing.assert_array_equal(snap.save(), before)
        src.store_host(100, K[100:], V[100:])
        assert not np.array_equal(src.save(), before)
        np.testing.assert_array_equal(snap.save(), before)
        snap.copy_to(src)
        np.testing.assert_array_equal(src.save(), before)
        with pytest.raises(pkg.XtgError):
            src.copy_to(other)
    finally:
        for c in (src, snap, other):
            c.destroy()

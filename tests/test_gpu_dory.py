"""GPU parity of the decode-step composition (xtg_hip_dory_*) against the oracle's (packs/dory/dory.cpp:467-578),
on the same seeded random-init weights and inputs.

Bars: logits rel-L2 <= 1e-3 and the same argmax per row (the parity bounds of the decode step), step after step; a
graph replay of a step gives the eager step's logits exactly.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def rel_l2(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(np.asarray(y, np.float64) - ref) / np.linalg.norm(ref))


def unit_rows(rng, m, h):
    x = rng.standard_normal((m, h)).astype(np.float32)
    return x / np.linalg.norm(x, axis=1, keepdims=True)


def test_tiny_model_many_steps(hip, orc, wl):
    """Two loops (per-loop caches), chunks of 8 then decode and verify steps: 12 prefill chunks wrap the 64-slot
    sliding rings; every call's logits are compared."""
    w = wl.DoryWeights(wl.DORY_TINY, seed=3, context=256)
    ref = orc.Dory(w, wl)
    dev = hip.dory(w)
    rng = np.random.default_rng(4)
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    dx = hip.array(shape=(8, H))
    dl = hip.array(shape=(8, V))
    pos = 0
    worst = 0.0
    for step, m in enumerate([8] * 12 + [1, 1, 8, 3, 1]):
        x = unit_rows(rng, m, H)
        dx.upload(np.concatenate([x, np.zeros((8 - m, H), np.float32)]))
        dev.forward(dx, m, pos, dl)
        got = dl.numpy()[:m]
        want = ref.forward(x, pos)
        e = rel_l2(got, want)
        worst = max(worst, e)
        assert e <= 1e-3, (step, e)
        assert (got.argmax(1) == want.argmax(1)).all(), step
        pos += m
    dx.free()
    dl.free()
    dev.destroy()
    print("tiny model: worst logits rel-L2 %.2e over %d positions" % (worst, pos))


@pytest.mark.parametrize("loops", [2, 1])
def test_one_token_steps_fused_and_separate(hip, orc, wl, monkeypatch, loops):
    """One-token steps run their norms inside the projections (records of partial sums); XTG_DECODE_UNFUSED=1 takes
    the separate norm launches instead. Both against the oracle, and against each other, over the same calls. With
    one loop the loop's entry and exit norms ride on the next projection too."""
    w = wl.DoryWeights(dict(wl.DORY_TINY, loops=loops), seed=13, context=128)
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    ref = orc.Dory(w, wl)
    fused = hip.dory(w)
    monkeypatch.setenv("XTG_DECODE_UNFUSED", "1")
    separate = hip.dory(w)
    monkeypatch.delenv("XTG_DECODE_UNFUSED")
    rng = np.random.default_rng(14)
    dx = hip.array(shape=(8, H))
    dl = hip.array(shape=(8, V))
    pos = 0
    for step, m in enumerate([8, 1, 1, 1, 3, 1, 1]):
        x = unit_rows(rng, m, H)
        dx.upload(np.concatenate([x, np.zeros((8 - m, H), np.float32)]))
        outs = []
        for dev in (fused, separate):
            dev.forward(dx, m, pos, dl)
            outs.append(dl.numpy()[:m].copy())
        want = ref.forward(x, pos)
        for got in outs:
            assert rel_l2(got, want) <= 1e-3, step
            assert (got.argmax(1) == want.argmax(1)).all(), step
        assert rel_l2(outs[0], outs[1]) <= 1e-4, step
        pos += m
    dx.free()
    dl.free()
    fused.destroy()
    separate.destroy()


@pytest.mark.parametrize("shape", [(1024, 2048, 8, 2), (1280, 2816, 10, 5)])
def test_verify_steps_split_and_whole_k(hip, orc, wl, monkeypatch, shape):
    """Steps of 2..8 rows split the gate/up, down and o projections' K in two (two output sets, added by the norm
    launch that reads them); XTG_VERIFY_WHOLE_K=1 keeps the whole K. Models wide enough that each half holds
    several k-tiles of 256 (hidden 1024, FFN 2048, 8 q heads of 128), and with odd k-tile counts, whose second half
    is a tile shorter (hidden 1280 and 10 q heads of 128: 5 tiles; FFN 2816: 11): both against the oracle, and
    against each other over the same calls (the halves' sum differs from the whole sum by rounding only); one-row
    steps between them."""
    hidden, ffn, heads, kv_heads = shape
    w = wl.DoryWeights(dict(wl.DORY_TINY, hidden=hidden, ffn=ffn, heads=heads, kv_heads=kv_heads, head_dim=128),
                       seed=15, context=128)
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    ref = orc.Dory(w, wl)
    split = hip.dory(w)
    monkeypatch.setenv("XTG_VERIFY_WHOLE_K", "1")
    whole = hip.dory(w)
    monkeypatch.delenv("XTG_VERIFY_WHOLE_K")
    rng = np.random.default_rng(16)
    dx = hip.array(shape=(8, H))
    dl = hip.array(shape=(8, V))
    pos = 0
    for step, m in enumerate([8, 2, 1, 5, 8, 3]):
        x = unit_rows(rng, m, H)
        dx.upload(np.concatenate([x, np.zeros((8 - m, H), np.float32)]))
        outs = []
        for dev in (split, whole):
            dev.forward(dx, m, pos, dl)
            outs.append(dl.numpy()[:m].copy())
        want = ref.forward(x, pos)
        for got in outs:
            assert rel_l2(got, want) <= 1e-3, step
            assert (got.argmax(1) == want.argmax(1)).all(), step
        e = rel_l2(outs[0], outs[1])
        print("step %d (%d rows): split against whole K %.2e" % (step, m, e))
        assert e <= 1e-4, step
        pos += m
    dx.free()
    dl.free()
    split.destroy()
    whole.destroy()


def test_wide_model_one_token_steps(hip, orc, wl, monkeypatch):
    """hidden 5120 / FFN 9728 with 32 q heads of 128: the q/k/v/g launch (640 row-blocks, 40 k-tiles) and the down
    projection (76 k-tiles) take launch shapes no fused one-token kernel is made for, so the session runs its
    one-token steps on the separate norm launches: bit for bit those of an XTG_DECODE_UNFUSED=1 session, and within
    the decode bar of the oracle."""
    cfg = dict(wl.DORY_TINY, hidden=5120, ffn=9728, heads=32, kv_heads=8, head_dim=128, n_in=2, n_rec=2, n_out=2,
               loops=1, window=16, ring_slots=24)
    w = wl.DoryWeights(cfg, seed=31, context=64)
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    ref = orc.Dory(w, wl)
    wide = hip.dory(w)
    monkeypatch.setenv("XTG_DECODE_UNFUSED", "1")
    separate = hip.dory(w)
    monkeypatch.delenv("XTG_DECODE_UNFUSED")
    rng = np.random.default_rng(32)
    dx = hip.array(shape=(8, H))
    dl = hip.array(shape=(8, V))
    pos = 0
    for step, m in enumerate([8, 1, 1, 3, 1]):
        x = unit_rows(rng, m, H)
        dx.upload(np.concatenate([x, np.zeros((8 - m, H), np.float32)]))
        outs = []
        for dev in (wide, separate):
            dev.forward(dx, m, pos, dl)
            outs.append(dl.numpy()[:m].copy())
        want = ref.forward(x, pos)
        np.testing.assert_array_equal(outs[0], outs[1])
        assert rel_l2(outs[0], want) <= 1e-3, step
        assert (outs[0].argmax(1) == want.argmax(1)).all(), step
        pos += m
    dx.free()
    dl.free()
    wide.destroy()
    separate.destroy()


def fill_context(w, ctx, oracle_model, dev_model, hip, rng):
    """Synthetic context: unit-norm K / V per head for positions 0 .. ctx - 1 in every global cache, and the last
    ring_slots of them in every sliding ring, the same rows on both sides."""
    c = w.cfg
    kvh, d, ring = c["kv_heads"], c["head_dim"], c["ring_slots"]
    K = wl_unit(rng, (ctx, kvh), d)
    Vv = wl_unit(rng, (ctx, kvh), d)
    a = 0
    for l, kind in enumerate(w.kinds):
        if kind == 0:
            continue
        lo = 0 if kind == 2 else max(0, ctx - ring)
        recurrent = c["n_in"] <= l < c["n_in"] + c["n_rec"]
        per_loop = c.get("kv_mode", 0) == 0
        for inst in range(c["loops"] if recurrent and per_loop else 1):   # per-loop caches of a recurrent sublayer
            oc = oracle_model.cache(a, inst)
            dc = dev_model.cache(a, inst)
            for p in range(lo, ctx, 1024):
                q = min(ctx, p + 1024)
                oc.store(p, K[p:q], Vv[p:q])
                dc.store_host(p, K[p:q], Vv[p:q])
        a += 1


def wl_unit(rng, shape, d):
    x = rng.standard_normal(tuple(shape) + (d,)).astype(np.float32)
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


@pytest.fixture(scope="module")
def model_4b(hip, orc, wl):
    ctx = 4096
    w = wl.DoryWeights(wl.DORY_4B, seed=5, context=ctx + 64)
    ref = orc.Dory(w, wl)
    dev = hip.dory(w)
    fill_context(w, ctx, ref, dev, hip, np.random.default_rng(6))
    yield w, ref, dev, ctx
    dev.destroy()


@pytest.mark.parametrize("m", [1, 8])
def test_4b_decode_step(hip, model_4b, m):
    """The synthetic 4B-shaped model at a 4K context: one decode (m = 1) or verify (m = 8) step of all 48
    sublayers."""
    w, ref, dev, ctx = model_4b
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    x = unit_rows(np.random.default_rng(7 + m), m, H)
    dx = hip.array(x)
    dl = hip.array(shape=(m, V))
    dev.forward(dx, m, ctx, dl)
    got = dl.numpy()
    want = ref.forward(x, ctx, threads=16)
    dx.free()
    dl.free()
    e = rel_l2(got, want)
    print("4B step m=%d: logits rel-L2 %.2e" % (m, e))
    assert e <= 1e-3
    assert (got.argmax(1) == want.argmax(1)).all()


@pytest.fixture(scope="module")
def model_real(hip, orc, wl):
    ctx = 4096
    w = wl.DoryWeights(wl.DORY_REAL, seed=91, context=ctx + 64)
    ref = orc.Dory(w, wl)
    dev = hip.dory(w)
    fill_context(w, ctx, ref, dev, hip, np.random.default_rng(92))
    yield w, ref, dev, ctx
    dev.destroy()


@pytest.mark.parametrize("m", [1, 8])
def test_real_dory_shape_step(hip, model_real, m):
    """The real Dory 4B's shape (hidden 2560, FFN 7168, 16 q / 4 KV heads of 256, 72 sublayers, two loops, FP8
    caches in last_loop mode, BF16 head) at a 4K context: a decode and a verify step against the oracle."""
    w, ref, dev, ctx = model_real
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    x = unit_rows(np.random.default_rng(90 + m), m, H)
    dx = hip.array(x)
    dl = hip.array(shape=(m, V))
    dev.forward(dx, m, ctx, dl)
    got = dl.numpy()
    want = ref.forward(x, ctx, threads=16)
    dx.free()
    dl.free()
    e = rel_l2(got, want)
    print("real Dory shape, step m=%d at 4K: logits rel-L2 %.2e" % (m, e))
    assert e <= 1e-3
    assert (got.argmax(1) == want.argmax(1)).all()


@pytest.fixture(scope="module")
def model_4b_8k(hip, orc, wl):
    ctx = 8192
    w = wl.DoryWeights(wl.DORY_4B, seed=81, context=ctx + 64)
    ref = orc.Dory(w, wl)
    dev = hip.dory(w)
    fill_context(w, ctx, ref, dev, hip, np.random.default_rng(82))
    yield w, ref, dev, ctx
    dev.destroy()


@pytest.mark.parametrize("m", [1, 8])
def test_4b_decode_step_8k(hip, model_4b_8k, m):
    """The synthetic 4B-shaped model at an 8K context: 16 splits per KV head on the global layers."""
    w, ref, dev, ctx = model_4b_8k
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    x = unit_rows(np.random.default_rng(80 + m), m, H)
    dx = hip.array(x)
    dl = hip.array(shape=(m, V))
    dev.forward(dx, m, ctx, dl)
    got = dl.numpy()
    want = ref.forward(x, ctx, threads=16)
    dx.free()
    dl.free()
    e = rel_l2(got, want)
    print("4B step at 8K m=%d: logits rel-L2 %.2e" % (m, e))
    assert e <= 1e-3
    assert (got.argmax(1) == want.argmax(1)).all()


@pytest.fixture(scope="module")
def model_4b_32k(hip, orc, wl):
    ctx = 32768
    w = wl.DoryWeights(wl.DORY_4B, seed=8, context=ctx + 64)
    ref = orc.Dory(w, wl)
    dev = hip.dory(w)
    fill_context(w, ctx, ref, dev, hip, np.random.default_rng(9))
    yield w, ref, dev, ctx
    dev.destroy()


@pytest.mark.parametrize("m", [1, 8])
def test_4b_decode_step_32k(hip, model_4b_32k, m):
    """The synthetic 4B-shaped model at a 32K context (the benchmark's longest): 32 splits per KV head on the
    global layers, the sliding rings wrapped many times over."""
    w, ref, dev, ctx = model_4b_32k
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    x = unit_rows(np.random.default_rng(70 + m), m, H)
    dx = hip.array(x)
    dl = hip.array(shape=(m, V))
    dev.forward(dx, m, ctx, dl)
    got = dl.numpy()
    want = ref.forward(x, ctx, threads=16)
    dx.free()
    dl.free()
    e = rel_l2(got, want)
    print("4B step at 32K m=%d: logits rel-L2 %.2e" % (m, e))
    assert e <= 1e-3
    assert (got.argmax(1) == want.argmax(1)).all()


def test_4b_graph_replay_matches_eager(hip, model_4b):
    """A captured step replays the eager step exactly, replay after replay, with eager work in between."""
    w, ref, dev, ctx = model_4b
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    x = unit_rows(np.random.default_rng(9), 8, H)
    dx = hip.array(x)
    dl = hip.array(shape=(8, V))
    dev.forward(dx, 8, ctx, dl)
    eager = dl.numpy()
    hip.graph_begin()
    dev.forward(dx, 8, ctx, dl)
    g = hip.graph_end("dory_step")
    for rep in range(3):
        dl.upload(np.zeros((8, V), np.float32))
        hip.graph_launch(g)
        np.testing.assert_array_equal(dl.numpy(), eager)
        dev.forward(dx, 1, ctx, dl)   # eager work between replays
        hip.finish()
    hip.graph_destroy(g)
    dx.free()
    dl.free()


def test_graph_per_position(hip, wl):
    """A captured step is the step at the captured position (its RoPE angles, cache slots and scan plan are launch
    arguments), so a decode loop captures one graph per position: twin sessions with the same history, one eager,
    one replaying a graph captured at each new position, give identical logits token after token."""
    w = wl.DoryWeights(wl.DORY_TINY, seed=21, context=128)
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    eager, graphed = hip.dory(w), hip.dory(w)
    rng = np.random.default_rng(22)
    dx = hip.array(shape=(8, H))
    la, lb = hip.array(shape=(8, V)), hip.array(shape=(8, V))
    for p in range(0, 24, 8):
        dx.upload(unit_rows(rng, 8, H))
        eager.forward(dx, 8, p, la)
        graphed.forward(dx, 8, p, lb)
    for p in range(24, 30):
        dx.upload(np.concatenate([unit_rows(rng, 1, H), np.zeros((7, H), np.float32)]))
        eager.forward(dx, 1, p, la)
        hip.graph_begin()
        graphed.forward(dx, 1, p, lb)
        g = hip.graph_end("step_at_%d" % p)
        hip.graph_launch(g)
        np.testing.assert_array_equal(lb.numpy()[:1], la.numpy()[:1])
        hip.graph_launch(g)   # a second replay at the same position rewrites the same slots
        np.testing.assert_array_equal(lb.numpy()[:1], la.numpy()[:1])
        hip.graph_destroy(g)
    dx.free()
    la.free()
    lb.free()
    eager.destroy()
    graphed.destroy()


def sharpened(w, seed=9):
    """q scaled up 40x and lr ~ U(0.3, 0.7): attention that depends on positions and masks (see
    tests/test_oracle_dory.py)."""
    rng = np.random.default_rng(seed)
    for L in w.layers:
        if "qscale" in L:
            L["qscale"] *= np.float32(40)
        L["lr"][:] = rng.uniform(0.3, 0.7, L["lr"].shape).astype(np.float32)
    return w


def device_steps(hip, w, x, pos0, chunk):
    dev = hip.dory(w)
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    dx = hip.array(shape=(8, H))
    dl = hip.array(shape=(8, V))
    out = []
    try:
        for r in range(0, x.shape[0], chunk):
            m = min(chunk, x.shape[0] - r)
            dx.upload(np.concatenate([x[r:r + m], np.zeros((8 - m, H), np.float32)]))
            dev.forward(dx, m, pos0 + r, dl)
            out.append(dl.numpy()[:m])
    finally:
        dx.free()
        dl.free()
        dev.destroy()
    return np.concatenate(out)


def test_sharp_chunks_and_steps(hip, orc, wl):
    """A sharp-attention tiny model over 72 positions (the rings wrap): device chunks of 8 and device one-row
    steps against the oracle's, and against each other (equal up to the BF16 rounding of cached keys)."""
    w = sharpened(wl.DoryWeights(wl.DORY_TINY, seed=21, context=256))
    x = unit_rows(np.random.default_rng(2), 72, w.cfg["hidden"])
    ref = orc.Dory(w, wl)
    want8 = np.concatenate([ref.forward(x[r:r + 8], r) for r in range(0, 72, 8)])
    ref1 = orc.Dory(w, wl)
    want1 = np.concatenate([ref1.forward(x[r:r + 1], r) for r in range(72)])
    got8 = device_steps(hip, w, x, 0, 8)
    got1 = device_steps(hip, w, x, 0, 1)
    e8, e1, ec = rel_l2(got8, want8), rel_l2(got1, want1), rel_l2(got8, got1)
    bar8, dec8 = sharp_bar(orc, wl, w, x, 8, want8)
    bar1, dec1 = sharp_bar(orc, wl, w, x, 1, want1)
    print("sharp tiny model: chunks %.2e (bar %.2e, %d of 72 rows decided), steps %.2e (bar %.2e, %d decided) vs the "
          "oracle; chunks vs steps %.2e" % (e8, bar8, dec8.sum(), e1, bar1, dec1.sum(), ec))
    assert e8 <= bar8 and e1 <= bar1
    assert dec8.mean() >= MIN_DECIDED and dec1.mean() >= MIN_DECIDED
    assert (got8.argmax(1) == want8.argmax(1))[dec8].all() and (got1.argmax(1) == want1.argmax(1))[dec1].all()
    assert ec < 1e-2


def test_sharp_one_token_steps_fused_equal_separate(hip, orc, wl, monkeypatch):
    """The sharpened tiny model's one-token steps on the fused path (norms riding on the projections) against the
    separate norm launches (XTG_DECODE_UNFUSED=1), over 48 positions that wrap the rings: the two differ only by
    FP32 rounding of the norms, so they must agree within the oracle's own change under a 1-ulp perturbation of its
    inputs (no 3x margin, no 1e-3 floor), with the same argmax on every decided row."""
    w = sharpened(wl.DoryWeights(wl.DORY_TINY, seed=26, context=128))
    x = unit_rows(np.random.default_rng(27), 48, w.cfg["hidden"])
    fused = device_steps(hip, w, x, 0, 1)
    monkeypatch.setenv("XTG_DECODE_UNFUSED", "1")
    separate = device_steps(hip, w, x, 0, 1)
    monkeypatch.delenv("XTG_DECODE_UNFUSED")
    want = oracle_steps(orc, wl, w, x, 1)
    ulp = np.random.default_rng(1).choice([-1.0, 1.0], x.shape).astype(np.float32) * np.float32(2.0 ** -23)
    moved = oracle_steps(orc, wl, w, (x * (1 + ulp)).astype(np.float32), 1)
    noise = rel_l2(moved, want)
    top2 = np.sort(want, axis=1)[:, -2:]
    decided = (top2[:, 1] - top2[:, 0]) > 3 * np.abs(moved - want).max(axis=1)
    e = rel_l2(fused, separate)
    print("sharp one-token steps: fused vs separate %.2e, the oracle's 1-ulp change %.2e, %d of %d rows decided"
          % (e, noise, decided.sum(), len(decided)))
    assert e <= max(noise, 1e-6)
    assert decided.mean() >= MIN_DECIDED
    assert (fused.argmax(1) == separate.argmax(1))[decided].all()


def test_window_one_chunks_equal_steps(hip, wl):
    """Window 1 (every attention sees only its own row): device chunks and steps agree to FP32 rounding."""
    w = sharpened(wl.DoryWeights(dict(wl.DORY_TINY, window=1), seed=23, context=64))
    for i, k in enumerate(w.kinds):
        if k == wl.FULL:
            w.kinds[i] = wl.SLIDING
            w.layers[i]["kind"] = wl.SLIDING
    x = unit_rows(np.random.default_rng(3), 8, w.cfg["hidden"])
    assert rel_l2(device_steps(hip, w, x, 0, 8), device_steps(hip, w, x, 0, 1)) < 1e-5


def test_ring_smaller_than_window_plus_chunk(hip, orc, wl):
    """Window 60 in 64-slot rings with chunks of 8: storing before the scan would overwrite keys the chunk's
    first rows still see, so the step stores after it (the reference's order); logits against the oracle, on the
    sharpened model's noise-floor bar (sharp_bar)."""
    w = sharpened(wl.DoryWeights(dict(wl.DORY_TINY, window=60), seed=24, context=128))
    x = unit_rows(np.random.default_rng(5), 96, w.cfg["hidden"])
    want = oracle_steps(orc, wl, w, x, 8)
    got = device_steps(hip, w, x, 0, 8)
    e = rel_l2(got, want)
    bar, decided = sharp_bar(orc, wl, w, x, 8, want)
    print("ring 64 / window 60 chunks of 8: logits rel-L2 %.2e (bar %.2e), %d of %d rows decided"
          % (e, bar, decided.sum(), len(decided)))
    assert e <= bar
    assert decided.mean() >= MIN_DECIDED
    assert (got.argmax(1) == want.argmax(1))[decided].all()


def oracle_steps(orc, wl, w, x, chunk):
    ref = orc.Dory(w, wl)
    return np.concatenate([ref.forward(x[r:r + chunk], r) for r in range(0, x.shape[0], chunk)])


def noise_bar(run_oracle, x, want):
    """The parity bar of a sharpened model, whose logits move by ~1e-4 when its FP32 inputs move by one ulp: 3x
    the oracle's own change under a 1-ulp perturbation of the input rows (at least 1e-3), and the rows whose argmax
    is decided at that precision: the top-2 margin above 3x the row's largest 1-ulp change. run_oracle(x) gives the
    oracle's logits of the same calls on other input rows."""
    ulp = np.random.default_rng(1).choice([-1.0, 1.0], x.shape).astype(np.float32) * np.float32(2.0 ** -23)
    wp = run_oracle((x * (1 + ulp)).astype(np.float32))
    top2 = np.sort(want, axis=1)[:, -2:]
    decided = (top2[:, 1] - top2[:, 0]) > 3 * np.abs(wp - want).max(axis=1)
    return max(1e-3, 3 * rel_l2(wp, want)), decided


# the least fraction of rows whose argmax a sharpened model's test compares (rows decided at the oracle's precision)
MIN_DECIDED = 0.9


def sharp_bar(orc, wl, w, x, chunk, want):
    return noise_bar(lambda xx: oracle_steps(orc, wl, w, xx, chunk), x, want)


@pytest.mark.parametrize("window,chunk", [(48, 8), (48, 1), (60, 8)])
def test_fp8_caches_chunks_and_steps(hip, orc, wl, window, chunk):
    """FP8 KV caches (the reference Dory's default, dory.cpp:141) in a tiny model over 72 positions: chunks of 8
    and one-row steps with window 48 (the producer quantises each row's own key into the cache before the scan)
    and window 60 in 64-slot rings (the store follows the scan); logits against the oracle's FP8 caches.
    Default scales: rel-L2 <= 1e-3. Sharpened (q x 40, lr ~ U(0.3, 0.7)) a key whose E4M3 rounding flips on a
    1-ulp difference upstream moves the logits by ~1e-3, so there the bar is 3x the oracle's own change when its
    inputs are perturbed by 1 ulp (about 1.4e-3, against 2.6e-4 with BF16 caches)."""
    for sharp in (False, True):
        w = wl.DoryWeights(dict(wl.DORY_TINY, window=window, kv_dtype=1), seed=25, context=128)
        if sharp:
            w = sharpened(w)
        x = unit_rows(np.random.default_rng(8), 72, w.cfg["hidden"])
        want = oracle_steps(orc, wl, w, x, chunk)
        got = device_steps(hip, w, x, 0, chunk)
        e = rel_l2(got, want)
        bar, decided = 1e-3, np.ones(len(want), bool)
        if sharp:
            bar, decided = sharp_bar(orc, wl, w, x, chunk, want)
        print("FP8 caches, window %d, chunks of %d, sharp %s: logits rel-L2 %.2e (bar %.2e), %d of %d rows decided"
              % (window, chunk, sharp, e, bar, decided.sum(), len(decided)))
        assert e <= bar
        assert decided.mean() >= MIN_DECIDED
        assert (got.argmax(1) == want.argmax(1))[decided].all()


def test_4b_decode_step_fp8(hip, orc, wl, model_4b):
    """The synthetic 4B-shaped model at a 4K context over FP8 caches: one verify step (m = 8) against the oracle's."""
    import copy
    w0, _, _, ctx = model_4b
    w = copy.copy(w0)
    w.cfg = dict(w0.cfg, kv_dtype=1)
    ref = orc.Dory(w, wl)
    dev = hip.dory(w)
    try:
        fill_context(w, ctx, ref, dev, hip, np.random.default_rng(6))
        H, V = w.cfg["hidden"], w.cfg["vocab"]
        x = unit_rows(np.random.default_rng(15), 8, H)
        dx = hip.array(x)
        dl = hip.array(shape=(8, V))
        dev.forward(dx, 8, ctx, dl)
        got = dl.numpy()
        want = ref.forward(x, ctx, threads=16)
        dx.free()
        dl.free()
    finally:
        dev.destroy()
    e = rel_l2(got, want)
    print("4B step m=8, FP8 caches: logits rel-L2 %.2e" % e)
    assert e <= 1e-3
    assert (got.argmax(1) == want.argmax(1)).all()


def test_fp8_global_gate_waves(hip, orc, wl, monkeypatch):
    """The one-token step's gate by heads over the global layer's split partials of an FP8 cache: 16, 32 and 64 key
    splits per KV head (17, 33 and 65 records per column at 4K, 8K and 32K positions) take one, two and four waves
    per head. An 8-sublayer model with the 4B attention shape (32 q / 8 KV heads of 128, one global layer, three
    1088-slot rings), the global cache filled to 32768 and the rings with the positions before each one-token step,
    at 4096, 8192 and 32768: the fused session's launches name the gate's wave count, and its logits agree with the
    separate norm launches' (XTG_DECODE_UNFUSED=1, whose gate merges all records in one work-group per row) within
    1e-4 and with the oracle's within 1e-3, same argmax."""
    cfg = dict(wl.DORY_4B, n_in=2, n_rec=4, n_out=2, vocab=4096, kv_dtype=1)
    ctx = 32768
    w = wl.DoryWeights(cfg, seed=91, context=ctx + 64)
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    ref = orc.Dory(w, wl)
    fused = hip.dory(w)
    monkeypatch.setenv("XTG_DECODE_UNFUSED", "1")
    separate = hip.dory(w)
    monkeypatch.delenv("XTG_DECODE_UNFUSED")
    rng = np.random.default_rng(92)
    K = wl_unit(rng, (ctx, cfg["kv_heads"]), cfg["head_dim"])
    Vv = wl_unit(rng, (ctx, cfg["kv_heads"]), cfg["head_dim"])

    def store(kind, lo, hi):   # positions lo .. hi - 1 into every cache of that kind, in all three sessions
        a = 0
        for k in w.kinds:
            if k == 0:
                continue
            if k == kind:
                for p in range(lo, hi, 1024):
                    q = min(hi, p + 1024)
                    ref.cache(a, 0).store(p, K[p:q], Vv[p:q])
                    fused.cache(a, 0).store_host(p, K[p:q], Vv[p:q])
                    separate.cache(a, 0).store_host(p, K[p:q], Vv[p:q])
            a += 1

    store(2, 0, ctx)   # the global cache: a step at pos reads positions below pos only
    dx = hip.array(shape=(1, H))
    dl = hip.array(shape=(1, V))
    try:
        for pos, waves in ((4096, 1), (8192, 2), (32768, 4)):
            store(1, pos - cfg["ring_slots"], pos)   # the rings: the slots' worth of positions before the step
            x = unit_rows(rng, 1, H)
            dx.upload(x)
            hip.profile(True, launches=True)
            fused.forward(dx, 1, pos, dl)
            _, launches = hip.profile_report(launches=True)
            hip.profile(False)
            got = dl.numpy().copy()
            separate.forward(dx, 1, pos, dl)
            sep = dl.numpy().copy()
            want = ref.forward(x, pos, threads=16)
            names = {n for n, _ in launches if n.startswith("attn_gate_heads_kernel")}
            assert "attn_gate_heads_kernel<128, %d>" % waves in names, (pos, sorted(names))
            e_sep, e_ref = rel_l2(got, sep), rel_l2(got, want)
            print("FP8 global gate at %d: %s; fused vs separate %.2e, vs oracle %.2e" % (pos, sorted(names), e_sep,
                                                                                     e_ref))
            assert e_sep <= 1e-4, pos
            assert e_ref <= 1e-3, pos
            assert (got.argmax(1) == want.argmax(1)).all() and (sep.argmax(1) == want.argmax(1)).all(), pos
    finally:
        dx.free()
        dl.free()
        fused.destroy()
        separate.destroy()


def test_bf16_head_and_fp8_caches(hip, orc, wl):
    """The BF16 checkpoint's configuration (dory.cpp:141, 325, 1203): a BF16 LM head over FP8 caches, the tiny
    model over 24 positions in chunks of 8 and single rows; logits against the oracle with the same head."""
    w = wl.DoryWeights(dict(wl.DORY_TINY, kv_dtype=1), seed=27, context=64)
    head = wl.f32_to_bf16(np.random.default_rng(28).standard_normal((w.cfg["vocab"], w.cfg["hidden"]),
                                                                     dtype=np.float32))
    x = unit_rows(np.random.default_rng(29), 24, w.cfg["hidden"])
    ref = orc.Dory(w, wl)
    ref.set_head_bf16(head)
    want = np.concatenate([ref.forward(x[r:r + 8], r) for r in range(0, 16, 8)] +
                          [ref.forward(x[r:r + 1], r) for r in range(16, 24)])
    dev = hip.dory(w)
    dev.set_head_bf16(head)
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    dx, dl = hip.array(shape=(8, H)), hip.array(shape=(8, V))
    got = []
    try:
        for r, m in [(0, 8), (8, 8)] + [(p, 1) for p in range(16, 24)]:
            dx.upload(np.concatenate([x[r:r + m], np.zeros((8 - m, H), np.float32)]))
            dev.forward(dx, m, r, dl)
            got.append(dl.numpy()[:m])
    finally:
        dx.free()
        dl.free()
        dev.destroy()
    got = np.concatenate(got)
    e = rel_l2(got, want)
    print("BF16 head, FP8 caches: logits rel-L2 %.2e" % e)
    assert e <= 1e-3
    assert (got.argmax(1) == want.argmax(1)).all()


@pytest.mark.parametrize("kv_dtype,sharp,parts", [(0, False, "2"), (0, True, "2"), (1, False, "2"), (0, False, "1")])
def test_tiny_prefill_chunks_then_steps(hip, pkg, orc, wl, monkeypatch, kv_dtype, sharp, parts):
    """The prefill path (chunks of more than 8 rows: GEMM projections, the many-row attention with its own-key
    tiles, the store after the scan) on the tiny model: prefill() over 700 rows in chunks of 512 + 188 with
    logits for every row, then four one-row steps, against the oracle's chunks of the same sizes. The 64-slot
    rings take whole chunks (a ring keeps a chunk's last 64 rows). parts = 1: the GEMMs take the single-part
    operand (XTG_GEMM_PARTS=1)."""
    monkeypatch.setenv("XTG_GEMM_PARTS", parts)
    w = wl.DoryWeights(dict(wl.DORY_TINY, kv_dtype=kv_dtype), seed=31 + kv_dtype, context=800)
    if sharp:
        w = sharpened(w, seed=32)
    H, V, n = w.cfg["hidden"], w.cfg["vocab"], 700
    x = unit_rows(np.random.default_rng(33), n + 4, H)
    def run_oracle(xx):
        ref = orc.Dory(w, wl)
        return np.concatenate([ref.forward(xx[0:512], 0, threads=16), ref.forward(xx[512:n], 512, threads=16)] +
                              [ref.forward(xx[p:p + 1], p) for p in range(n, n + 4)])

    want = run_oracle(x)
    dev = hip.dory(w)
    dx, dl = hip.array(x[:n]), hip.array(shape=(n, V))
    dx1, dl1 = hip.array(shape=(1, H)), hip.array(shape=(1, V))
    got = []
    try:
        dev.prefill(dx, n, 0, pkg.LOGITS_ALL, dl)
        got.append(dl.numpy())
        for p in range(n, n + 4):
            dx1.upload(x[p:p + 1])
            dev.forward(dx1, 1, p, dl1)
            got.append(dl1.numpy())
    finally:
        for a in (dx, dl, dx1, dl1):
            a.free()
        dev.destroy()
    got = np.concatenate(got)
    e = rel_l2(got, want)
    bar, decided = noise_bar(run_oracle, x, want) if sharp else (1e-3, np.ones(len(want), bool))
    print("tiny prefill 512 + 188 rows then steps (KV dtype %d, sharp %s, %s parts): logits rel-L2 %.2e (bar %.2e), %d "
          "of %d rows decided" % (kv_dtype, sharp, parts, e, bar, decided.sum(), len(decided)))
    assert e <= bar
    assert decided.mean() >= MIN_DECIDED
    assert (got.argmax(1) == want.argmax(1))[decided].all()


def test_tiny_prefill_logits_last_and_none(hip, pkg, orc, wl):
    """prefill() with logits for the last row only (one row of the second chunk: its own operand), and with none
    followed by a step, against the oracle."""
    w = wl.DoryWeights(wl.DORY_TINY, seed=35, context=1400)
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    x = unit_rows(np.random.default_rng(36), 1201, H)
    ref = orc.Dory(w, wl)
    want_last = None
    for r in range(0, 600, 512):
        want_last = ref.forward(x[r:min(600, r + 512)], r, threads=16)[-1]
    for r in range(600, 1200, 512):
        ref.forward(x[r:min(1200, r + 512)], r, threads=16)
    want_step = ref.forward(x[1200:1201], 1200)[0]
    dev = hip.dory(w)
    dx, dl = hip.array(x), hip.array(shape=(1, V))
    try:
        dev.prefill(dx, 600, 0, pkg.LOGITS_LAST, dl)
        got_last = dl.numpy()[0]
        dev.prefill(dx.ptr + 600 * H * 4, 600, 600, pkg.LOGITS_NONE)   # rows 600 .. 1199 of x
        dev.forward(dx.ptr + 1200 * H * 4, 1, 1200, dl)
        got_step = dl.numpy()[0]
    finally:
        dx.free()
        dl.free()
        dev.destroy()
    for got, want in ((got_last, want_last), (got_step, want_step)):
        assert rel_l2(got, want) <= 1e-3
        assert got.argmax() == want.argmax()


def test_4b_prefill_chunk(hip, orc, model_4b):
    """The synthetic 4B-shaped model at a 4K context: one 40-row chunk (five operand groups on the GEMM, five attention row
    blocks) against the oracle's."""
    w, ref, dev, ctx = model_4b
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    x = unit_rows(np.random.default_rng(41), 40, H)
    dx = hip.array(x)
    dl = hip.array(shape=(40, V))
    dev.forward(dx, 40, ctx, dl)
    got = dl.numpy()
    want = ref.forward(x, ctx, threads=16)
    dx.free()
    dl.free()
    e = rel_l2(got, want)
    print("4B chunk of 40 rows: logits rel-L2 %.2e" % e)
    assert e <= 1e-3
    assert (got.argmax(1) == want.argmax(1)).all()


@pytest.mark.parametrize("kv_dtype", [0, 1])
def test_snapshot_restore_rings(hip, wl, kv_dtype):
    """Snapshot slot 0 after a 200-row prompt, run a step, run 100 more rows (the 64-slot rings lose the keys the
    step needs), restore slot 0 and run the step again: the logits equal the first run's exactly. Without the
    restore they differ."""
    w = wl.DoryWeights(dict(wl.DORY_TINY, kv_dtype=kv_dtype), seed=45, context=400)
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    x = unit_rows(np.random.default_rng(46), 308, H)
    dev = hip.dory(w)
    dx, dl = hip.array(x), hip.array(shape=(8, V))
    step = dx.ptr + 200 * H * 4   # rows 200 .. 207
    try:
        dev.prefill(dx, 200, 0, 0)
        dev.snapshot(0)
        dev.forward(step, 8, 200, dl)
        first = dl.numpy()
        dev.prefill(dx.ptr + 208 * H * 4, 100, 208, 0)
        dev.forward(step, 8, 200, dl)
        stale = dl.numpy()
        dev.restore(0)
        dev.forward(step, 8, 200, dl)
        again = dl.numpy()
    finally:
        dx.free()
        dl.free()
        dev.destroy()
    np.testing.assert_array_equal(again, first)
    assert rel_l2(stale, first) > 1e-4

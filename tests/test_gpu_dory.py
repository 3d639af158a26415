"""GPU parity of the decode-step composition (xtg_hip_dory_*) against the oracle's (packs/dory/dory.cpp:467-578),
on the same seeded random-init weights and inputs.

Bars: logits rel-L2 <= 1e-3 and the same argmax per row (the north star's bounds), step after step; a graph
replay of a step gives the eager step's logits exactly.
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
        for inst in range(c["loops"] if recurrent else 1):   # per-loop caches of a recurrent sublayer
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
    """Config 4 at a 4K context: one decode (m = 1) or verify (m = 8) step of the full 48-sublayer model."""
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

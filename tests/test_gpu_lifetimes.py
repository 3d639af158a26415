"""Device memory lifetimes around graphs and shared weights (xtier-go_amd/csrc/backend.cpp):

- a graph captured before a larger call grows the backend's scratch (a 512-row prefill chunk needs more attention
  partials and operand space than an 8-row step) still replays exactly: the outgrown buffers are kept while a graph
  exists;
- two sessions on the same host weights share the prepared device copies; destroying the one that prepared them
  leaves the other running (its logits unchanged), and the shared weights cannot be released from under it.
Each test opens a backend of its own, so its scratch starts empty."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def unit_rows(rng, m, h):
    x = rng.standard_normal((m, h)).astype(np.float32)
    return x / np.linalg.norm(x, axis=1, keepdims=True)


def test_graph_replay_after_scratch_growth(pkg, wl):
    b = pkg.HipBackend(0)
    try:
        w = wl.DoryWeights(wl.DORY_TINY, seed=31, context=1024)
        dev = b.dory(w)
        H, V = w.cfg["hidden"], w.cfg["vocab"]
        rng = np.random.default_rng(32)
        dx = b.array(unit_rows(rng, 8, H))
        dl = b.array(shape=(8, V))
        dev.forward(dx, 8, 0, dl)   # sizes the scratch for 8 rows
        eager = dl.numpy()
        b.graph_begin()
        dev.forward(dx, 8, 0, dl)
        g = b.graph_end("step8")
        # a 512-row chunk at positions 8 .. 519 outgrows the scratch the graph captured
        big = b.array(unit_rows(rng, 512, H))
        big_logits = b.array(shape=(512, V))
        dev.forward(big, 512, 8, big_logits)
        b.finish()
        for rep in range(3):
            dl.upload(np.zeros((8, V), np.float32))
            b.graph_launch(g)
            # the step at position 0 sees no cached key (every stored position is >= 0): its own keys only
            np.testing.assert_array_equal(dl.numpy(), eager)
            dev.forward(big, 512, 8, big_logits)   # eager work of the larger shape between replays
            b.finish()
        b.graph_destroy(g)
        for a in (dx, dl, big, big_logits):
            a.free()
        dev.destroy()
    finally:
        b.close()


def test_sessions_share_prepared_weights(pkg, wl, orc):
    b = pkg.HipBackend(0)
    try:
        w = wl.DoryWeights(wl.DORY_TINY, seed=33, context=256)
        H, V = w.cfg["hidden"], w.cfg["vocab"]
        x = unit_rows(np.random.default_rng(34), 4, H)
        want = orc.Dory(w, wl).forward(x, 0)
        first = b.dory(w)    # prepares every weight
        second = b.dory(w)   # finds them prepared
        dx = b.array(x)
        dl = b.array(shape=(4, V))
        with pytest.raises(pkg.XtgError, match="in use by a Dory session"):
            b.release_weight(pkg.Weight(*w.layers[0]["q"]))
        first.destroy()
        second.forward(dx, 4, 0, dl)
        got = dl.numpy()
        e = float(np.linalg.norm(got.astype(np.float64) - want) / np.linalg.norm(want.astype(np.float64)))
        assert e <= 1e-3 and (got.argmax(1) == want.argmax(1)).all(), e
        second.destroy()
        # no session holds them now: the caller may release them
        b.release_weight(pkg.Weight(*w.layers[0]["q"]))
        dx.free()
        dl.free()
    finally:
        b.close()

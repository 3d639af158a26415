"""Properties of the oracle's decode-step composition (packs/dory/dory.cpp:467-578), which cannot be run against
the reference itself here (DorySession needs the whole engine, safetensors loading and OpenCL to build).

- lr = 0 makes every sublayer return its normalised input (slerp at its first endpoint, kernels.cpp:177-189), and
  the loop entry / exit norms keep the direction (dory.cpp:530-541): the logits are then the head of the input
  row times logit_scale, up to the norm's epsilon.
- Causality and the cache: a chunk of m rows at pos0 gives the same logits as m one-row steps at pos0 .. pos0 +
  m - 1 (up to the BF16 rounding of keys that are cached in one case and still FP32 in the other); a one-position
  slip of the steps, a plausible bookkeeping mistake, fails the same bound by more than an order of magnitude.
- With a window of 1 no key but a row's own is visible, so chunks and steps agree to FP32 rounding.
"""
import numpy as np
import pytest


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def unit_rows(rng, m, h):
    x = rng.standard_normal((m, h)).astype(np.float32)
    return x / np.linalg.norm(x, axis=1, keepdims=True)


def sharpened(w, seed=9):
    """Weights whose attention matters: q scaled up 40x (sharp softmax, so positions and masks change the output)
    and lr ~ U(0.3, 0.7) (each sublayer moves x by a lot). A random model with the default scales attends
    almost uniformly and a position slip barely shows."""
    rng = np.random.default_rng(seed)
    for L in w.layers:
        if "qscale" in L:
            L["qscale"] *= np.float32(40)
        L["lr"][:] = rng.uniform(0.3, 0.7, L["lr"].shape).astype(np.float32)
    return w


@pytest.fixture(scope="module")
def tiny(wl):
    return sharpened(wl.DoryWeights(wl.DORY_TINY, seed=21, context=256))


def test_lr_zero_is_identity(orc, wl, tiny):
    w = wl.DoryWeights(wl.DORY_TINY, seed=22, context=64)
    for L in w.layers:
        L["lr"][:] = 0.0
    model = orc.Dory(w, wl)
    x = unit_rows(np.random.default_rng(1), 3, w.cfg["hidden"])
    got = model.forward(x, 0)
    (head,) = orc.matmul_nvfp4([w.head], x)
    want = head * w.logit_scale
    # the direction is kept exactly up to rounding; the length shrinks by the norms' epsilon (1e-6 per norm)
    f = float((got.astype(np.float64) * want).sum() / (want.astype(np.float64) ** 2).sum())
    assert abs(f - 1.0) < 1e-4
    assert rel_l2(got, f * want) < 1e-5


def steps(orc, wl, w, x, pos0, chunk):
    model = orc.Dory(w, wl)
    out = []
    for r in range(0, x.shape[0], chunk):
        out.append(model.forward(x[r:r + chunk], pos0 + r))
    return np.concatenate(out)


def test_chunk_equals_steps(orc, wl, tiny):
    """72 positions (the 64-slot rings wrap) as chunks of 8 and as 72 one-row steps."""
    x = unit_rows(np.random.default_rng(2), 72, tiny.cfg["hidden"])
    a = steps(orc, wl, tiny, x, 0, 8)
    b = steps(orc, wl, tiny, x, 0, 1)
    e = rel_l2(a, b)
    assert e < 1e-2, e
    # a one-position slip of the single-row steps (RoPE angles, cache slots and masks all shifted)
    c = steps(orc, wl, tiny, x, 1, 1)
    assert rel_l2(c, b) > 10 * max(e, 1e-2)


def test_window_edge(orc, wl, tiny):
    """A row exactly one window past a key no longer sees it: with the window shrunk to 1 every attention
    sublayer sees only its own row, so chunked and one-row runs agree to FP32 rounding (no BF16 keys involved)."""
    w = sharpened(wl.DoryWeights(dict(wl.DORY_TINY, window=1), seed=23, context=64))
    for i, k in enumerate(w.kinds):   # global sublayers would still see everything: make them sliding
        if k == wl.FULL:
            w.kinds[i] = wl.SLIDING
            w.layers[i]["kind"] = wl.SLIDING
    x = unit_rows(np.random.default_rng(3), 8, w.cfg["hidden"])
    a = steps(orc, wl, w, x, 0, 8)
    b = steps(orc, wl, w, x, 0, 1)
    assert rel_l2(a, b) < 1e-5

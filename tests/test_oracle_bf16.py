"""The oracle's matmul_bf16 (engine/src/kernels.cpp:140-155: each BF16 weight row to FP32, then an FP32 dot with
every input row), pinned by:
- the golden vectors written by the compiled reference (tests/golden/bf16_k*.npz), at <= 1e-6 relative;
- the compiled reference itself (oracle/_ref) where it is built, on a larger case;
- an FP64 closed form of the same product: max |err| / RMS <= 3e-5 (tests/opencl_test.cpp:57's bar), which a
  transposed weight, a dropped last input or a truncated (not rounded) BF16 weight fail.
"""
import glob
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def f64_ref(w_bits, x):
    w = (w_bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return x.astype(np.float64) @ w.T


def err_rms(y, ref):
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / np.sqrt(np.mean(ref ** 2)))


def test_golden(orc):
    files = sorted(glob.glob(os.path.join(GOLDEN, "bf16_k*.npz")))
    assert len(files) == 2
    for f in files:
        d = np.load(f)
        for m in (1, 3, 8):
            y = orc.matmul_bf16(d["w"], d["x%d" % m], threads=3)
            want = d["y%d" % m]
            assert np.max(np.abs(y - want)) <= 1e-6 * np.sqrt(np.mean(want.astype(np.float64) ** 2)), (f, m)


def test_closed_form_and_planted_mistakes(orc, wl):
    rng = np.random.default_rng(3)
    k = 1024
    w = wl.f32_to_bf16(rng.standard_normal((k, k)).astype(np.float32))
    x = rng.uniform(-1, 1, (4, k)).astype(np.float32)
    ref = f64_ref(w, x)
    assert err_rms(orc.matmul_bf16(w, x), ref) <= 3e-5
    # a transposed weight
    assert err_rms(orc.matmul_bf16(np.ascontiguousarray(w.T), x), ref) > 1e-1
    # the last input dropped
    x2 = x.copy()
    x2[:, -1] = 0
    assert err_rms(orc.matmul_bf16(w, x2), ref) > 1e-3
    # weights truncated from FP32 instead of rounded: the closed form of the rounded weights tells them apart
    wf = rng.standard_normal((64, k)).astype(np.float32)
    rounded = wl.f32_to_bf16(wf)
    truncated = (wf.view(np.uint32) >> 16).astype(np.uint16)
    assert (rounded != truncated).any()
    assert err_rms(orc.matmul_bf16(truncated, x), f64_ref(rounded, x)) > 3e-5


def test_against_reference(orc, wl):
    if not orc.ref_available():
        pytest.skip("oracle/_ref is not built here (no reference tree)")
    rng = np.random.default_rng(4)
    w = wl.f32_to_bf16(rng.standard_normal((700, 2560)).astype(np.float32))
    for m in (1, 2, 8):
        x = rng.standard_normal((m, 2560)).astype(np.float32)
        a = orc.matmul_bf16(w, x, threads=4)
        b = orc.matmul_bf16(w, x, threads=4, use_ref=True)
        assert np.max(np.abs(a - b)) <= 1e-6 * np.sqrt(np.mean(b.astype(np.float64) ** 2))

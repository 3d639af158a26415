"""The oracle's matmul_nvfp4 (engine/src/kernels.cpp:84-138), pinned by:
- an FP64 closed form over the dense decoded weights (tests/kernels_test.cpp:57-87's check, error / RMS < 2e-5);
- the dense decode written independently in numpy (workloads.decode_nvfp4) against the oracle's nvfp4_row;
- a planted mistake (a dropped group scale) that the closed-form check must catch;
- the compiled reference (oracle/_ref) where it exists: equal to within 1e-6 of the RMS output;
- committed golden vectors (tests/golden/nvfp4_*.npz) written by tests/golden/make_golden.py from oracle/_ref.
"""
import glob
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def random_weight(rng, n, k, glob=0.37):
    # tests/kernels_test.cpp:43-55: random code bytes, positive normal E4M3 scales 0x20..0x4f, global 0.37
    codes = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = (0x20 + rng.integers(0, 0x30, size=(n, k // 16))).astype(np.uint8)
    return codes, scales, glob


def err_over_rms(y, ref):
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / np.sqrt(np.mean(ref ** 2)))


def test_nvfp4_row_equals_numpy_decode(orc, wl):
    rng = np.random.default_rng(1)
    codes, scales, g = random_weight(rng, 9, 256)
    dense = wl.decode_nvfp4(codes, scales, g)
    for n in range(9):
        np.testing.assert_array_equal(orc.nvfp4_row(codes, scales, g, n), dense[n])


@pytest.mark.parametrize("m", [1, 2, 7])
def test_matmul_vs_fp64(orc, wl, m):
    """tests/kernels_test.cpp:57-87: two fused weights (70 x 256, 33 x 256), m in {1, 2, 7} (both branches)."""
    rng = np.random.default_rng(42 + m)
    a = random_weight(rng, 70, 256)
    b = random_weight(rng, 33, 256)
    x = rng.uniform(-1, 1, size=(m, 256)).astype(np.float32)
    ya, yb = orc.matmul_nvfp4([a, b], x)
    for (codes, scales, g), y in ((a, ya), (b, yb)):
        ref = x.astype(np.float64) @ wl.decode_nvfp4(codes, scales, g).astype(np.float64).T
        assert err_over_rms(y, ref) < 2e-5


def test_closed_form_catches_dropped_scale(orc, wl):
    """A plausible mistake -- one group scale left out -- must fail the closed-form bar."""
    rng = np.random.default_rng(3)
    codes, scales, g = random_weight(rng, 40, 256)
    x = rng.uniform(-1, 1, size=(1, 256)).astype(np.float32)
    (y,) = orc.matmul_nvfp4([(codes, scales, g)], x)
    wrong = wl.decode_nvfp4(codes, scales, g).astype(np.float64)
    wrong[:, 16:32] /= wl.E4M3[scales[:, 1]].astype(np.float64)[:, None]   # group 1 without its scale
    assert err_over_rms(y, x.astype(np.float64) @ wrong.T) > 1e-3


@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_matmul_config_shapes_vs_fp64(orc, wl, m):
    """The benchmark distributions (uniform codes, |N(0,1)|*0.05 scales, unit BF16 rows) at K = N = 3072."""
    rng = np.random.default_rng(100 + m)
    codes, scales, g = wl.nvfp4_weight(rng, 3072, 3072)
    x = wl.bf16_to_f32(wl.unit_rows_bf16(rng, m, 3072))
    (y,) = orc.matmul_nvfp4([(codes, scales, g)], x)
    ref = x.astype(np.float64) @ wl.decode_nvfp4(codes, scales, g).astype(np.float64).T
    assert err_over_rms(y, ref) < 2e-5


def test_matmul_rejects_bad_widths(orc):
    rng = np.random.default_rng(4)
    a = random_weight(rng, 4, 256)
    b = random_weight(rng, 4, 128)
    with pytest.raises(ValueError):
        orc.matmul_nvfp4([a, b], np.zeros((1, 256), np.float32))


@pytest.mark.skipif(not __import__("oracle").ref_available(), reason="oracle/_ref not built (no reference tree)")
@pytest.mark.parametrize("m", [1, 2, 3, 7, 8])
def test_matmul_vs_reference(orc, wl, m):
    rng = np.random.default_rng(200 + m)
    a = wl.nvfp4_weight(rng, 300, 3072)
    b = random_weight(rng, 33, 3072)
    x = rng.uniform(-1, 1, size=(m, 3072)).astype(np.float32)
    mine = orc.matmul_nvfp4([a, b], x)
    ref = orc.matmul_nvfp4([a, b], x, use_ref=True, threads=4)
    for y, r in zip(mine, ref):
        assert err_over_rms(y, r) <= 1e-6


def test_matmul_golden(orc):
    files = sorted(glob.glob(os.path.join(GOLDEN, "nvfp4_*.npz")))
    assert files, "no golden NVFP4 vectors committed"
    for f in files:
        d = np.load(f)   # allow_pickle stays False
        ws = []
        i = 0
        while "codes%d" % i in d:
            ws.append((d["codes%d" % i], d["scales%d" % i], float(d["glob%d" % i])))
            i += 1
        ys = orc.matmul_nvfp4(ws, d["x"])
        for i, y in enumerate(ys):
            assert err_over_rms(y, d["y%d" % i]) <= 1e-6, f

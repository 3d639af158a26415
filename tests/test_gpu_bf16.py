"""GPU parity of the BF16 GEMV / skinny GEMM (include/xtg_hip.h xtg_hip_matmul_bf16*) against the oracle's
matmul_bf16 (engine/src/kernels.cpp:140-155) on the same seeded inputs.

Bars: rel-L2 <= 1e-5 against the oracle and the golden vectors; max |err| / RMS <= 3e-5 against the FP64 closed
form (tests/opencl_test.cpp:57's device bar). Shapes: the golden k = 320 and k = 260 (k % 8 == 4), ragged row
counts, every row count 1..8 (one and two column blocks of activation terms), more than 8 rows through the host
call, and the LM head of the BF16 checkpoint (131072 x 2560, packs/dory/dory.cpp:325) at M = 1 and 8.
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


def err_over_rms(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / np.sqrt(np.mean(ref ** 2)))


def exact(w, x):
    return x.astype(np.float64) @ (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64).T


def weight(wl, rng, n, k):
    return wl.f32_to_bf16(rng.standard_normal((n, k), dtype=np.float32))


def device_matmul(hip, w, x, x_dtype=0):
    m = x.shape[0]
    dx = hip.array(x)
    dy = hip.array(shape=(m, w.shape[0]))
    hip.matmul_bf16_dev(w, dx, x_dtype, m, dy)
    y = dy.numpy()
    dx.free()
    dy.free()
    return y


def test_golden_vectors(hip):
    files = sorted(glob.glob(os.path.join(GOLDEN, "bf16_k*.npz")))
    assert files
    for f in files:
        d = np.load(f)
        w = np.ascontiguousarray(d["w"])
        for m in (1, 3, 8):
            x, want = d["x%d" % m], d["y%d" % m]
            assert rel_l2(hip.matmul_bf16(w, x), want) <= 1e-5, (f, m)
            assert rel_l2(device_matmul(hip, w, x), want) <= 1e-5, (f, m)
            assert err_over_rms(device_matmul(hip, w, x), exact(w, x)) <= 3e-5, (f, m)
        hip.release_bf16(w)


@pytest.mark.parametrize("n,k", [(1, 4), (17, 36), (40, 264), (129, 1032), (300, 4100)])
def test_ragged_shapes(hip, orc, wl, n, k):
    """Row counts that do not fill a 16-row block; k a multiple of 4 but not of 8 or 128."""
    rng = np.random.default_rng(n * 1000 + k)
    w = weight(wl, rng, n, k)
    for m in (1, 5, 6, 8):
        x = rng.standard_normal((m, k)).astype(np.float32)
        y = device_matmul(hip, w, x)
        assert rel_l2(y, orc.matmul_bf16(w, x)) <= 1e-5, (m, n, k)
        assert err_over_rms(y, exact(w, x)) <= 3e-5, (m, n, k)
    hip.release_bf16(w)


def test_every_row_count(hip, orc, wl):
    """m = 1..8 on a 4096 x 3072 weight (one column block of activation terms up to 5 rows, two above)."""
    rng = np.random.default_rng(11)
    w = weight(wl, rng, 4096, 3072)
    x = rng.standard_normal((8, 3072)).astype(np.float32)
    for m in range(1, 9):
        y = device_matmul(hip, w, x[:m])
        assert rel_l2(y, orc.matmul_bf16(w, x[:m])) <= 1e-5, m
    hip.release_bf16(w)


def test_host_call_many_rows_and_bf16_input(hip, orc, wl):
    """19 rows through the host-synchronous call (passes of 8); BF16 activations on the device call."""
    rng = np.random.default_rng(12)
    w = weight(wl, rng, 1000, 640)
    x = rng.standard_normal((19, 640)).astype(np.float32)
    assert rel_l2(hip.matmul_bf16(w, x), orc.matmul_bf16(w, x)) <= 1e-5
    xb = wl.f32_to_bf16(x[:8])
    y = device_matmul(hip, w, np.ascontiguousarray(xb), x_dtype=1)
    assert rel_l2(y, orc.matmul_bf16(w, wl.bf16_to_f32(xb))) <= 1e-5
    hip.release_bf16(w)


@pytest.mark.parametrize("m", [1, 8])
def test_lm_head_shape(hip, orc, wl, m):
    """The BF16 checkpoint's LM head, 131072 x 2560 (671 MB), unit-norm rows; argmax per row matches too."""
    rng = np.random.default_rng(13 + m)
    w = weight(wl, rng, 131072, 2560)
    x = rng.standard_normal((m, 2560)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    y = device_matmul(hip, w, x)
    ref = orc.matmul_bf16(w, x, threads=16)
    hip.release_bf16(w)
    assert rel_l2(y, ref) <= 1e-5
    assert (y.argmax(1) == ref.argmax(1)).all()


def test_errors(hip, pkg):
    w = np.zeros((8, 6), np.uint16)
    with pytest.raises(pkg.XtgError, match="k % 4"):
        hip.prepare_bf16(w)
    w = np.zeros((8, 8), np.uint16)
    with pytest.raises(pkg.XtgError, match="rows"):
        dx = hip.array(shape=(9, 8))
        dy = hip.array(shape=(9, 8))
        try:
            hip.matmul_bf16_dev(w, dx, 0, 9, dy)
        finally:
            dx.free()
            dy.free()

"""The reference's own device test (tests/opencl_test.cpp:16-93) through the host-synchronous entries: NVFP4 weights
70x256, 7168x2560 and 2560x7168 (random code bytes, scales 0x20 + r % 48, global 0.37), x uniform over
{-1, -0.999, ..., 1}; a decode projection fused four times equals itself and the single projection bit for bit;
M in {1, 2, 7, 65, 512} checked at 32 sampled columns of the first and last row against FP64 dots of the decoded
weight rows, max |err| / RMS < 3e-5; the BF16 head 131072x2560 at M in {1, 2, 16} likewise."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def sampled_err(y, x, wrows, cols, rows):
    err, sq, cnt = 0.0, 0.0, 0
    for r in rows:
        ref = wrows.astype(np.float64) @ x[r].astype(np.float64)
        got = y[r, cols].astype(np.float64)
        err = max(err, float(np.max(np.abs(ref - got))))
        sq += float(np.sum(ref * ref))
        cnt += len(cols)
    return err / np.sqrt(sq / cnt)


@pytest.mark.parametrize("n,k", [(70, 256), (7168, 2560), (2560, 7168)])
def test_opencl_real_shapes(hip, pkg, wl, n, k):
    rng = np.random.default_rng(42 + n)
    codes = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = (0x20 + rng.integers(0, 48, size=(n, k // 16))).astype(np.uint8)
    w = pkg.Weight(codes, scales, np.float32(0.37))

    def rnd(shape):
        return ((rng.integers(0, 2001, size=shape) - 1000) / 1000).astype(np.float32)

    x = rnd((1, k))
    a, b, c, d = hip.matmul([w, w, w, w], x)
    assert np.array_equal(a, b) and np.array_equal(a, c) and np.array_equal(a, d)
    (s,) = hip.matmul([w], x)
    assert np.array_equal(a, s)
    cols = np.array([(j * 137 + 3) % n for j in range(32)])
    wrows = wl.decode_nvfp4(codes[cols], scales[cols], np.float32(0.37))
    for m in (1, 2, 7, 65, 512):
        x = rnd((m, k))
        (y,) = hip.matmul([w], x)
        e = sampled_err(y, x, wrows, cols, (0, m - 1))
        print("NVFP4 M=%d N=%d K=%d err/RMS %.2e" % (m, n, k, e))
        assert e < 3e-5


def test_opencl_bf16_head(hip, wl):
    n, k = 131072, 2560
    rng = np.random.default_rng(7)
    w = wl.f32_to_bf16(((rng.integers(0, 2001, size=(n, k)) - 1000) / 1000).astype(np.float32))
    cols = np.array([(j * 4093 + 3) % n for j in range(32)])
    wrows = wl.bf16_to_f32(w[cols])
    for m in (1, 2, 16):
        x = ((rng.integers(0, 2001, size=(m, k)) - 1000) / 1000).astype(np.float32)
        y = hip.matmul_bf16(w, x)
        e = sampled_err(y, x, wrows, cols, (0, m - 1))
        print("BF16 M=%d N=%d K=%d err/RMS %.2e" % (m, n, k, e))
        assert e < 3e-5

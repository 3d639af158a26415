"""GPU parity of the NVFP4 GEMV / skinny GEMM (include/xtg_hip.h xtg_hip_matmul_nvfp4*) against the oracle's
matmul_nvfp4 (engine/src/kernels.cpp:84-138) on the same seeded inputs.

Bars: rel-L2 <= 1e-5 against the oracle; max |err| / RMS <= 3e-5 against the FP64 closed form (the reference's
own device bar, tests/opencl_test.cpp:57). Shapes: the reference unit test's fused 70x256 + 33x256, ragged row
counts, K not a multiple of 128, and the config shapes (3072x3072, QKV 5120, gate/up 2x8192, down K=8192) at
M in {1, 2, 4, 8}.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def rel_l2(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(np.asarray(y, np.float64) - ref) / np.linalg.norm(ref))


def err_over_rms(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / np.sqrt(np.mean(ref ** 2)))


def kt_weight(rng, n, k):
    codes = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = (0x20 + rng.integers(0, 0x30, size=(n, k // 16))).astype(np.uint8)
    return codes, scales, 0.37


@pytest.mark.parametrize("m", [1, 2, 7, 8, 13])
def test_unit_shapes_host_call(hip, pkg, orc, wl, m):
    """tests/kernels_test.cpp:57-87 shapes through the host-synchronous entry (rows > 8 run in passes of 8)."""
    rng = np.random.default_rng(42 + m)
    a, b = kt_weight(rng, 70, 256), kt_weight(rng, 33, 256)
    x = rng.uniform(-1, 1, size=(m, 256)).astype(np.float32)
    ys = hip.matmul([pkg.Weight(*a), pkg.Weight(*b)], x)
    refs = orc.matmul_nvfp4([a, b], x)
    for y, r, w in zip(ys, refs, (a, b)):
        assert rel_l2(y, r) <= 1e-5
        exact = x.astype(np.float64) @ wl.decode_nvfp4(*w).astype(np.float64).T
        assert err_over_rms(y, exact) <= 3e-5


@pytest.mark.parametrize("n,k", [(1, 16), (17, 48), (40, 272), (129, 1040)])
def test_ragged_shapes(hip, pkg, orc, n, k):
    """Row counts that do not fill a 16-row block, K a multiple of 16 but not of 32 or 128."""
    rng = np.random.default_rng(n * 1000 + k)
    w = kt_weight(rng, n, k)
    for m in (1, 3, 8):
        x = rng.standard_normal((m, k)).astype(np.float32)
        (y,) = hip.matmul([pkg.Weight(*w)], x)
        (r,) = orc.matmul_nvfp4([w], x)
        assert rel_l2(y, r) <= 1e-5, (m, n, k)


def test_zero_and_extreme_scales(hip, pkg, orc):
    """Zero scales (code 0x00), the largest scale 448 (0x7e) and the smallest subnormal 2^-9 (0x01)."""
    rng = np.random.default_rng(9)
    n, k = 64, 512
    codes = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = rng.choice(np.array([0x00, 0x01, 0x07, 0x38, 0x7E, 0x40], np.uint8), size=(n, k // 16))
    x = rng.standard_normal((4, k)).astype(np.float32)
    (y,) = hip.matmul([pkg.Weight(codes, scales, 1.0)], x)
    (r,) = orc.matmul_nvfp4([(codes, scales, 1.0)], x)
    assert rel_l2(y, r) <= 1e-5


def test_activation_scale_extremes(hip, pkg, orc):
    """Rows of very different magnitude (1e-30 .. 1e30): each row is brought into f16 range on its own."""
    rng = np.random.default_rng(10)
    w = kt_weight(rng, 48, 256)
    x = rng.standard_normal((4, 256)).astype(np.float32)
    x[0] *= 1e-30
    x[1] *= 1e30
    x[2, 5] = 3e4
    (y,) = hip.matmul([pkg.Weight(*w)], x)
    (r,) = orc.matmul_nvfp4([w], x)
    for i in range(4):
        assert rel_l2(y[i], r[i]) <= 1e-5, i


SHAPES = [(3072, 3072), (5120, 3072), (16384, 3072), (3072, 8192)]


@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_config_shapes_device_bf16(hip, pkg, orc, wl, n, k, m):
    """The config weights and BF16 unit rows through the device entry, x given as BF16."""
    rng = np.random.default_rng(n + k + m)
    w = wl.nvfp4_weight(rng, n, k)
    xb = wl.unit_rows_bf16(rng, m, k)
    x32 = wl.bf16_to_f32(xb)
    dx = hip.array(xb)
    dy = hip.array(shape=(m, n))
    hip.matmul_dev([pkg.Weight(*w)], dx, pkg.X_BF16, m, dy)
    y = dy.numpy()
    dx.free()
    dy.free()
    (r,) = orc.matmul_nvfp4([w], x32)
    assert rel_l2(y, r) <= 1e-5
    if m in (1, 8) and n <= 5120:
        exact = x32.astype(np.float64) @ wl.decode_nvfp4(*w).astype(np.float64).T
        assert err_over_rms(y, exact) <= 3e-5


def test_fused_gate_up_device_f32(hip, pkg, orc, wl):
    """gate/up as one fused call (the MLP's two projections into consecutive [m][n] blocks), FP32 x."""
    rng = np.random.default_rng(77)
    g = wl.nvfp4_weight(rng, 8192, 3072)
    u = wl.nvfp4_weight(rng, 8192, 3072)
    m = 8
    x = rng.standard_normal((m, 3072)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    dx = hip.array(x)
    dy = hip.array(np.full(16 + 2 * m * 8192, np.nan, dtype=np.float32))
    hip.matmul_dev([pkg.Weight(*g), pkg.Weight(*u)], dx, pkg.X_F32, m, dy, y_offset=16)
    y = dy.numpy()
    dx.free()
    dy.free()
    assert np.isnan(y[:16]).all()   # nothing written before y_offset
    rg, ru = orc.matmul_nvfp4([g, u], x)
    assert rel_l2(y[16:16 + m * 8192].reshape(m, 8192), rg) <= 1e-5
    assert rel_l2(y[16 + m * 8192:].reshape(m, 8192), ru) <= 1e-5


@pytest.mark.parametrize("xdt", ["f32", "bf16"])
@pytest.mark.parametrize("n,k", [(5120, 3072), (3072, 8192), (40, 272)])
def test_raw_rows_and_prepared_operand(hip, pkg, orc, wl, xdt, n, k):
    """The device entry reads FP32 / BF16 rows as they are where the launch shape allows (the GEMV builds each
    k-tile's operand with its own power of two) and otherwise prepares the operand first; both against the oracle,
    and so is the explicit two-step path (prep_x + matmul_op). Rows whose magnitude changes by 1e9 along k; rows
    that do not start on a 16-byte boundary are refused."""
    rng = np.random.default_rng(n + k)
    w = wl.nvfp4_weight(rng, n, k)
    for m in (1, 3, 8):
        x = rng.standard_normal((m, k)).astype(np.float32)
        x[0, :128] *= 1e6
        x[-1, k // 2:] *= 1e-3
        if xdt == "bf16":
            payload, dt = wl.f32_to_bf16(x).ravel(), pkg.X_BF16
            x = wl.bf16_to_f32(payload.reshape(m, k))
        else:
            payload, dt = x.ravel(), pkg.X_F32
        e = payload.dtype.itemsize
        pad = np.zeros(16 // e, payload.dtype)
        (r,) = orc.matmul_nvfp4([w], x)
        buf = hip.array(shape=(payload.size + pad.size,), dtype=payload.dtype)
        dy = hip.array(shape=(m, n))
        op = hip.array(shape=((m + 7) // 8 * hip.x_operand_bytes(k),), dtype=np.uint8)
        buf.upload(np.concatenate([payload, pad]))
        hip.matmul_dev([pkg.Weight(*w)], buf.ptr, dt, m, dy)
        assert rel_l2(dy.numpy(), r) <= 1e-5, (m, "aligned")
        hip.prep_x(buf.ptr, dt, m, k, op)
        hip.matmul_op([pkg.Weight(*w)], op, m, dy)
        assert rel_l2(dy.numpy(), r) <= 1e-5, (m, "two-step")
        with pytest.raises(pkg.XtgError):   # rows must start on a 16-byte boundary
            hip.matmul_dev([pkg.Weight(*w)], buf.ptr + e, dt, m, dy)
        for arr in (buf, dy, op):
            arr.free()


def test_fused_qkvg_four_weights(hip, pkg, orc, wl):
    """q / k / v / g of the attention sublayer (4096 + 1024 + 1024 + 4096 rows) in one launch."""
    rng = np.random.default_rng(78)
    ws = [wl.nvfp4_weight(rng, n, 3072) for n in (4096, 1024, 1024, 4096)]
    x = rng.standard_normal((3, 3072)).astype(np.float32)
    ys = hip.matmul([pkg.Weight(*w) for w in ws], x)
    refs = orc.matmul_nvfp4(ws, x)
    for y, r in zip(ys, refs):
        assert rel_l2(y, r) <= 1e-5


def test_errors_are_reported(hip, pkg):
    rng = np.random.default_rng(1)
    a = kt_weight(rng, 8, 256)
    b = kt_weight(rng, 8, 128)
    with pytest.raises(pkg.XtgError, match="widths differ"):
        hip.matmul([pkg.Weight(*a), pkg.Weight(*b)], np.zeros((1, 256), np.float32))
    with pytest.raises(pkg.XtgError, match="rows"):   # one device call takes at most 4096 rows
        hip.matmul_dev([pkg.Weight(*a)], 0, pkg.X_F32, 5000, 0)


def test_raw_bf16_tiny_and_nonfinite_rows(hip, pkg, orc, wl):
    """BF16 rows read raw: a row of BF16 subnormals and tiny normals (the tile exponent is capped), a row spanning
    2^-60 .. 2^60 within one tile, a zero row, and a row holding a NaN (its outputs are NaN; the other rows are
    untouched)."""
    rng = np.random.default_rng(12)
    n, k = 48, 384
    w = kt_weight(rng, n, k)
    x = rng.standard_normal((5, k)).astype(np.float32)
    x[0] *= np.float32(2.0 ** -128)
    x[1, ::2] *= np.float32(2.0 ** 60)
    x[1, 1::2] *= np.float32(2.0 ** -60)
    x[2] = 0.0
    x[4, 200] = np.nan
    xb = wl.f32_to_bf16(x)
    x = wl.bf16_to_f32(xb)
    dx, dy = hip.array(xb), hip.array(shape=(5, n))
    hip.matmul_dev([pkg.Weight(*w)], dx, pkg.X_BF16, 5, dy)
    y = dy.numpy()
    dx.free()
    dy.free()
    (r,) = orc.matmul_nvfp4([w], np.where(np.isnan(x), 0, x).astype(np.float32))
    for i in range(4):
        if i == 2:
            assert (y[i] == 0).all()
        else:
            assert rel_l2(y[i], r[i]) <= 1e-5, i
    assert np.isnan(y[4]).all()


@pytest.mark.parametrize("m", [1, 2])
def test_block_scaled_rows_edge_cases(hip, pkg, orc, wl, m):
    """One and two BF16 rows take the block-scaled FP4 x FP8 matrix op (each input split into two E4M3 parts at its
    16-input group's power of two). Rows built against that split: magnitudes from 2^-60 to 2^60 alternating within
    every group (the small half far below E4M3's range at the group's exponent: its contribution is below 2^-100 of
    the output), BF16 subnormals (the exponent cap), one group of exact zeros in an otherwise normal row, values
    whose 8 significant bits need both parts (128 + odd), magnitudes near 2^100, and -- in the last row of the
    two-row case -- an infinity and a NaN in separate groups (that row's outputs are NaN, the other row's are not).
    Against the oracle at rel-L2 1e-5 and the FP64 closed form at max |err| / RMS 3e-5."""
    rng = np.random.default_rng(31 + m)
    n, k = 272, 768
    w = kt_weight(rng, n, k)
    rows = []
    x = rng.standard_normal(k).astype(np.float32)
    x[::2] *= np.float32(2.0 ** 60)
    x[1::2] *= np.float32(2.0 ** -60)
    rows.append(x)
    rows.append((rng.standard_normal(k) * 2.0 ** -128).astype(np.float32))   # BF16 subnormals
    x = rng.standard_normal(k).astype(np.float32)
    x[32:48] = 0.0
    rows.append(x)
    rows.append(((rng.integers(0, 2, k) * 2 - 1) * (128 + 2 * rng.integers(0, 64, k) + 1)).astype(np.float32))
    rows.append((rng.standard_normal(k) * 2.0 ** 100).astype(np.float32))   # large, the FP32 sums stay finite
    for i, x in enumerate(rows):
        xs = [x] if m == 1 else [x, rows[(i + 1) % len(rows)]]
        xb = wl.f32_to_bf16(np.stack(xs))
        x32 = wl.bf16_to_f32(xb)
        dx, dy = hip.array(xb), hip.array(shape=(m, n))
        hip.matmul_dev([pkg.Weight(*w)], dx, pkg.X_BF16, m, dy)
        y = dy.numpy()
        dx.free()
        dy.free()
        (r,) = orc.matmul_nvfp4([w], x32)
        exact = x32.astype(np.float64) @ wl.decode_nvfp4(*w).astype(np.float64).T
        for j in range(m):
            assert np.isfinite(y[j]).all(), (i, j)
            assert rel_l2(y[j], r[j]) <= 1e-5, (i, j)
            assert err_over_rms(y[j], exact[j]) <= 3e-5, (i, j)
    if m == 2:
        x = rng.standard_normal((2, k)).astype(np.float32)
        x[1, 100] = np.inf
        x[1, 300] = np.nan
        xb = wl.f32_to_bf16(x)
        dx, dy = hip.array(xb), hip.array(shape=(2, n))
        hip.matmul_dev([pkg.Weight(*w)], dx, pkg.X_BF16, 2, dy)
        y = dy.numpy()
        dx.free()
        dy.free()
        (r,) = orc.matmul_nvfp4([w], wl.bf16_to_f32(xb[:1]))
        assert rel_l2(y[0], r[0]) <= 1e-5
        assert np.isnan(y[1]).all()


def tiles_np(codes, scales):
    """The documented tile layout: tile (rb, kt) holds lane l = 16 g + r's 16 code bytes (row rb * 16 + r, inputs
    kt * 128 + 32 g .. + 32) at 16 l and its two scale bytes at 1024 + 2 l; zeros past n and k."""
    n, k = codes.shape[0], codes.shape[1] * 2
    nb, kt = -(-n // 16), -(-k // 128)
    cp = np.zeros((nb * 16, kt * 64), np.uint8)
    cp[:n, :k // 2] = codes
    sp = np.zeros((nb * 16, kt * 8), np.uint8)
    sp[:n, :k // 16] = scales
    c = cp.reshape(nb, 16, kt, 4, 16).transpose(0, 2, 3, 1, 4).reshape(nb, kt, 1024)
    s = sp.reshape(nb, 16, kt, 4, 2).transpose(0, 2, 3, 1, 4).reshape(nb, kt, 128)
    return np.concatenate([c, s], axis=2).ravel()


@pytest.mark.parametrize("n,k", [(17, 48), (40, 272), (3072, 3072), (24576, 8192)])
def test_device_repack_matches_layout(hip, pkg, n, k):
    """prepare() copies the checkpoint's row-major arrays to the device and repacks them there (row-blocks at a
    time through a 64 MiB staging buffer: the last shape takes two chunks); the tiles equal the documented
    layout byte for byte."""
    rng = np.random.default_rng(n + k)
    codes = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = rng.integers(0, 127, size=(n, k // 16), dtype=np.uint8)
    w = pkg.Weight(codes, scales, 0.5)
    hip.prepare(w)
    got = hip.nvfp4_tiles(w)
    hip.release_weight(w)
    np.testing.assert_array_equal(got, tiles_np(codes, scales))

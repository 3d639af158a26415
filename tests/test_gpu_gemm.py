"""GPU parity of the NVFP4 GEMM for prefill chunks (more than 8 rows per device call, include/xtg_hip.h
xtg_hip_matmul_nvfp4_dev / _op) against the oracle's matmul_nvfp4 prefill branch (engine/src/kernels.cpp:116-137).

Bars: rel-L2 <= 1e-5 against the oracle; max |err| / RMS <= 3e-5 against the FP64 closed form. Shapes: the
layer projections at prefill chunk sizes (64 .. 512 rows), row counts that leave partial 8-row groups and partial
64-row tiles, ragged weights, four fused weights, every launch shape, and more rows than one host pass. The
single-part operand (XTG_GEMM_PARTS=1: each activation's high f16 part alone, the f16 precision of the reference's
GPU prefill GEMM) is held to rel-L2 <= 5e-4 and max |err| / RMS <= 3e-3 against the FP64 closed form.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def rel_l2(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(np.asarray(y, np.float64) - ref) / np.linalg.norm(ref))


def err_over_rms(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / np.sqrt(np.mean(ref ** 2)))


def device_matmul(hip, pkg, ws, x):
    m = x.shape[0]
    dx = hip.array(x)
    dy = hip.array(shape=(m * sum(w.n_out for w in ws),))
    hip.matmul_dev(ws, dx, pkg.X_F32, m, dy)
    y = dy.numpy()
    dx.free()
    dy.free()
    out, off = [], 0
    for w in ws:
        out.append(y[off:off + m * w.n_out].reshape(m, w.n_out))
        off += m * w.n_out
    return out


@pytest.mark.parametrize("name,n,k,m", [("qkv", 5120, 3072, 512), ("gateup", 8192, 3072, 64),
                                        ("down", 3072, 8192, 200), ("ragged", 129, 1040, 37),
                                        ("group_edge", 1000, 3072, 9), ("tile_edge", 2048, 512, 65)])
def test_shapes(hip, pkg, orc, wl, name, n, k, m):
    rng = np.random.default_rng(n + k + m)
    w = wl.nvfp4_weight(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    (y,) = device_matmul(hip, pkg, [pkg.Weight(*w)], x)
    (ref,) = orc.matmul_nvfp4([w], x)
    assert rel_l2(y, ref) <= 1e-5, name
    exact = x.astype(np.float64) @ wl.decode_nvfp4(*w).astype(np.float64).T
    assert err_over_rms(y, exact) <= 3e-5, name


def test_fused_weights(hip, pkg, orc, wl):
    """q / k / v / g of a 4B-shaped attention sublayer in one call (consecutive [m][n_i] blocks), 96 rows."""
    rng = np.random.default_rng(5)
    shapes = [(4096, 3072), (1024, 3072), (1024, 3072), (4096, 3072)]
    ws = [wl.nvfp4_weight(rng, n, k) for n, k in shapes]
    x = wl.bf16_to_f32(wl.unit_rows_bf16(rng, 96, 3072))
    ys = device_matmul(hip, pkg, [pkg.Weight(*w) for w in ws], x)
    for y, r in zip(ys, orc.matmul_nvfp4(ws, x)):
        assert rel_l2(y, r) <= 1e-5


@pytest.mark.parametrize("shape", ["4,4", "2,4", "1,4"])
def test_every_launch_shape(hip, pkg, orc, wl, shape):
    rng = np.random.default_rng(7)
    w = wl.nvfp4_weight(rng, 1200, 1024)
    x = rng.standard_normal((75, 1024)).astype(np.float32)
    os.environ["XTG_GEMM_SHAPE"] = shape
    try:
        (y,) = device_matmul(hip, pkg, [pkg.Weight(*w)], x)
    finally:
        del os.environ["XTG_GEMM_SHAPE"]
    (ref,) = orc.matmul_nvfp4([w], x)
    assert rel_l2(y, ref) <= 1e-5, shape


def test_host_call_more_rows_than_a_pass(hip, pkg, orc, wl):
    """600 rows through the host-synchronous call: passes of 512 and 88 rows."""
    rng = np.random.default_rng(8)
    w = wl.nvfp4_weight(rng, 700, 2048)
    x = rng.standard_normal((600, 2048)).astype(np.float32)
    (y,) = hip.matmul([pkg.Weight(*w)], x)
    (ref,) = orc.matmul_nvfp4([w], x)
    assert rel_l2(y, ref) <= 1e-5


def test_gemm_matches_gemv_rows(hip, pkg, wl):
    """The first 8 rows of a 16-row GEMM call against the GEMV on those 8 rows: the same operand and FP32 sums of
    the same products, so they agree to FP32 rounding."""
    rng = np.random.default_rng(9)
    w = pkg.Weight(*wl.nvfp4_weight(rng, 3072, 3072))
    x = rng.standard_normal((16, 3072)).astype(np.float32)
    (a,) = device_matmul(hip, pkg, [w], x)
    (b,) = device_matmul(hip, pkg, [w], x[:8])
    assert rel_l2(a[:8], b) <= 1e-6


@pytest.mark.parametrize("n,k,m", [(5120, 3072, 512), (8192, 3072, 2048), (3072, 8192, 200), (129, 1040, 37),
                                   (1000, 3072, 9), (2048, 512, 65), (700, 2048, 17)])
def test_single_part(hip, pkg, orc, wl, monkeypatch, n, k, m):
    """Row counts of one 8-row group past a pair (9, 17), partial pairs and tiles, the heuristic's shapes."""
    rng = np.random.default_rng(n * 3 + k + m)
    w = wl.nvfp4_weight(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    monkeypatch.setenv("XTG_GEMM_PARTS", "1")
    (y,) = device_matmul(hip, pkg, [pkg.Weight(*w)], x)
    exact = x.astype(np.float64) @ wl.decode_nvfp4(*w).astype(np.float64).T
    (ref,) = orc.matmul_nvfp4([w], x)
    assert rel_l2(y, ref) <= 5e-4
    assert rel_l2(y, exact) <= 5e-4
    assert err_over_rms(y, exact) <= 3e-3


@pytest.mark.parametrize("shape", ["4,4", "2,4", "1,4", "4,2", "2,2", "1,2"])
def test_single_part_every_launch_shape(hip, pkg, orc, wl, monkeypatch, shape):
    rng = np.random.default_rng(17)
    w = wl.nvfp4_weight(rng, 1200, 1024)
    x = rng.standard_normal((75, 1024)).astype(np.float32)
    monkeypatch.setenv("XTG_GEMM_PARTS", "1")
    monkeypatch.setenv("XTG_GEMM_SHAPE", shape)
    (y,) = device_matmul(hip, pkg, [pkg.Weight(*w)], x)
    exact = x.astype(np.float64) @ wl.decode_nvfp4(*w).astype(np.float64).T
    assert rel_l2(y, exact) <= 5e-4, shape
    assert err_over_rms(y, exact) <= 3e-3, shape


def test_single_part_fused_weights(hip, pkg, wl, monkeypatch):
    """q / k / v / g in one call with the single-part operand against the two-part one, 96 rows."""
    rng = np.random.default_rng(6)
    shapes = [(4096, 3072), (1024, 3072), (1024, 3072), (4096, 3072)]
    ws = [pkg.Weight(*wl.nvfp4_weight(rng, n, k)) for n, k in shapes]
    x = wl.bf16_to_f32(wl.unit_rows_bf16(rng, 96, 3072))
    two = device_matmul(hip, pkg, ws, x)
    monkeypatch.setenv("XTG_GEMM_PARTS", "1")
    one = device_matmul(hip, pkg, ws, x)
    for a, b in zip(one, two):
        assert rel_l2(a, b) <= 5e-4

"""Number formats of the oracle, pinned by the reference's known answers (tests/kernels_test.cpp:30-41), by the
OCP E4M3 / IEEE BF16 definitions written independently in numpy (xtier-go_amd/workloads.py), and against the
compiled reference (engine/src/fp.cpp) where oracle/_ref exists."""
import math

import numpy as np
import pytest


def test_e4m3_known_answers(orc):
    o = orc.oracle()
    # tests/kernels_test.cpp:31-39
    assert o.xo_e4m3_to_f32(0x38) == 1.0
    assert o.xo_e4m3_to_f32(0x7E) == 448.0
    assert o.xo_e4m3_to_f32(0x01) == math.ldexp(1.0, -9)
    assert math.isnan(o.xo_e4m3_to_f32(0x7F)) and math.isnan(o.xo_e4m3_to_f32(0xFF))
    for c in range(256):
        if (c & 0x7F) == 0x7F:
            continue
        assert o.xo_f32_to_e4m3(o.xo_e4m3_to_f32(c)) == c, c
    assert o.xo_f32_to_e4m3(1000.0) == 0x7E and o.xo_f32_to_e4m3(-1000.0) == 0xFE
    # tests/kernels_test.cpp:40
    assert o.xo_f32_to_bf16(1.0) == 0x3F80 and o.xo_bf16_to_f32(0x3F80) == 1.0


def test_e4m3_table_matches_definition(orc, wl):
    o = orc.oracle()
    table = np.array([o.xo_e4m3_to_f32(b) for b in range(256)], dtype=np.float32)
    np.testing.assert_array_equal(table, wl.E4M3)   # NaN positions compare equal in assert_array_equal


def test_e4m3_rounding_midpoints(orc):
    """Ties go to the even code; a value just above a midpoint rounds up (RNE by the definition)."""
    o = orc.oracle()
    for c in range(0, 0x7E):
        lo, hi = o.xo_e4m3_to_f32(c), o.xo_e4m3_to_f32(c + 1)
        mid = np.float32((np.float64(lo) + np.float64(hi)) / 2)
        if float(mid) * 2 != lo + hi:   # midpoint not representable in FP32: no tie to test
            continue
        want = c if c % 2 == 0 else c + 1
        assert o.xo_f32_to_e4m3(float(mid)) == want, (c, mid)
        assert o.xo_f32_to_e4m3(float(np.nextafter(mid, np.float32(1e9)))) == c + 1
        assert o.xo_f32_to_e4m3(float(np.nextafter(mid, np.float32(-1e9)))) == c


def test_e4m3_encoder_numpy_vs_oracle(orc, wl):
    o = orc.oracle()
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 0.05,
                        rng.standard_normal(2000).astype(np.float32) * 100,
                        (rng.random(2000) * 2 ** -8).astype(np.float32),
                        np.array([0.0, -0.0, 448.0, 449.0, 464.0, 1e30, -1e30, np.inf, -np.inf], np.float32)])
    got = wl.f32_to_e4m3(x)
    want = np.array([o.xo_f32_to_e4m3(float(v)) for v in x], dtype=np.uint8)
    np.testing.assert_array_equal(got, want)


def test_bf16_numpy_vs_oracle(orc, wl):
    o = orc.oracle()
    rng = np.random.default_rng(6)
    bits = rng.integers(0, 2 ** 32, size=5000, dtype=np.uint64).astype(np.uint32)
    bits = bits[(bits & 0x7F800000) != 0x7F800000]   # finite values (NaN payloads differ through ctypes floats)
    x = bits.view(np.float32)
    got = wl.f32_to_bf16(x)
    want = np.array([o.xo_f32_to_bf16(float(v)) for v in x], dtype=np.uint16)
    np.testing.assert_array_equal(got, want)


def test_kv_fp8_bits_match_table_rounding(orc):
    """engine/src/kv.cpp:19-40's bit-level E4M3 rounding equals the table search of fp.cpp:30-49 on every value
    below the saturation bound (both are round to nearest even)."""
    o = orc.oracle()
    rng = np.random.default_rng(7)
    x = np.concatenate([(rng.random(20000) * 460).astype(np.float32), (rng.random(5000) * 0.02).astype(np.float32)])
    x = np.concatenate([x, -x])
    for v in x:
        assert o.xo_e4m3_bits(float(v)) == o.xo_f32_to_e4m3(float(v)), v


@pytest.mark.skipif(not __import__("oracle").ref_available(), reason="oracle/_ref not built (no reference tree)")
def test_formats_vs_reference(orc):
    o, r = orc.oracle(), orc.ref()
    rng = np.random.default_rng(8)
    x = np.concatenate([rng.standard_normal(5000).astype(np.float32) * s for s in (1e-3, 0.05, 3.0, 300.0)])
    for v in x:
        assert o.xo_f32_to_e4m3(float(v)) == r.xr_f32_to_e4m3(float(v))
        assert o.xo_f32_to_bf16(float(v)) == r.xr_f32_to_bf16(float(v))
    for b in range(256):
        a, c = o.xo_e4m3_to_f32(b), r.xr_e4m3_to_f32(b)
        assert a == c or (math.isnan(a) and math.isnan(c))

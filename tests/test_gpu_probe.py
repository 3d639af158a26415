"""The streaming-read probe (xtg_hip_read_probe; the reference's readsum device probe, tests/gpu_probe.cpp:59-66)
against numpy: each work-group's XOR partial of its 32 KiB of 16-byte blocks, the last one partial."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 32768, 1 << 20, (1 << 20) + 48 * 16])
def test_read_probe_partials(hip, nbytes):
    rng = np.random.default_rng(nbytes)
    words = rng.integers(0, 1 << 32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    n = hip.read_probe_partials(nbytes)
    assert n == -(-nbytes // 32768)
    src = hip.array(words, dtype=np.uint32)
    out = hip.array(np.full(n, 0xDEADBEEF, np.uint32), dtype=np.uint32)
    hip.read_probe(src, nbytes, out)
    got = out.numpy()
    want = np.array([np.bitwise_xor.reduce(words[i * 8192:(i + 1) * 8192]) for i in range(n)], np.uint32)
    src.free()
    out.free()
    np.testing.assert_array_equal(got, want)

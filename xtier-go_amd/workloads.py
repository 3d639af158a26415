"""Seeded synthetic inputs for the decode-path workloads (numpy PCG64 streams, so every run and every machine
sees the same bytes).

NVFP4 weights: E2M1 codes uniform over all 16 codes (two per byte, low nibble first), one E4M3 scale per 16
inputs drawn as |N(0,1)| * 0.05 and rounded to E4M3 (nearest even, saturating), tensor scale 1.0.
Activations: rows drawn from N(0,1), L2-normalised, stored as BF16 (rounded to nearest even); the FP32 view of
those BF16 values is what an FP32 consumer receives.
"""
import numpy as np

# --------------------------------------------------------------------------------------------------- formats


def _e4m3_table():
    """Values of the 256 E4M3 (float8_e4m3fn) codes: bias 7, subnormal step 2^-9, 0x7f / 0xff NaN."""
    t = np.zeros(256, dtype=np.float32)
    for b in range(256):
        e, m = (b >> 3) & 15, b & 7
        if (b & 0x7F) == 0x7F:
            mag = np.nan
        elif e == 0:
            mag = m * 2.0 ** -9
        else:
            mag = (1 + m / 8) * 2.0 ** (e - 7)
        t[b] = -mag if b & 0x80 else mag
    return t


E4M3 = _e4m3_table()
E2M1 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6, -0.0, -0.5, -1, -1.5, -2, -3, -4, -6], dtype=np.float32)


def f32_to_e4m3(x):
    """FP32 -> E4M3 codes: the largest code not above |x|, then nearest even; |x| >= 448 saturates to 0x7e."""
    x = np.asarray(x, dtype=np.float32)
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.uint8)
    a = np.abs(x)
    pos = E4M3[:0x7F]   # codes 0x00 .. 0x7e, increasing
    lo = np.searchsorted(pos, a, side="right") - 1
    lo = np.clip(lo, 0, 0x7E)
    nxt = np.minimum(lo + 1, 0x7E)
    d0 = (a - pos[lo]).astype(np.float32)
    d1 = (pos[nxt] - a).astype(np.float32)
    up = (lo < 0x7E) & ((d1 < d0) | ((d1 == d0) & ((lo & 1) == 1)))
    code = (lo + up).astype(np.uint8)
    code = np.where(a >= 448.0, 0x7E, code).astype(np.uint8)
    code = np.where(np.isnan(x), 0x7F, code).astype(np.uint8)
    return (code | sign).astype(np.uint8)


def f32_to_bf16(x):
    """FP32 -> BF16 bits, round to nearest even (a NaN stays a quiet NaN)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = ((b + np.uint32(0x7FFF) + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((b >> 16) | 0x40).astype(np.uint16), r)


def bf16_to_f32(h):
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def decode_nvfp4(codes, scales, glob=1.0):
    """Dense FP32 [n][k] of an NVFP4 weight (the value each code stands for, scales folded in)."""
    n = codes.shape[0]
    lo = E2M1[codes & 15]
    hi = E2M1[codes >> 4]
    w = np.empty((n, codes.shape[1] * 2), dtype=np.float32)
    w[:, 0::2] = lo
    w[:, 1::2] = hi
    sc = np.repeat(E4M3[scales].astype(np.float32) * np.float32(glob), 16, axis=1)
    return w * sc


# -------------------------------------------------------------------------------------------------- weights


def nvfp4_weight(rng, n, k, scale_std=0.05, glob=1.0):
    """(codes [n][k/2] u8, scales [n][k/16] u8, global) with the distributions above."""
    codes = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    s = (np.abs(rng.standard_normal(size=(n, k // 16), dtype=np.float32)) * np.float32(scale_std)).astype(np.float32)
    return codes, f32_to_e4m3(s), float(glob)


def unit_rows_bf16(rng, m, k):
    """[m][k] BF16 bits of unit-norm rows (N(0,1), normalised in FP32, rounded to BF16)."""
    x = rng.standard_normal(size=(m, k), dtype=np.float32)
    x /= np.sqrt((x.astype(np.float64) ** 2).sum(axis=1, keepdims=True)).astype(np.float32)
    return f32_to_bf16(x)


def unit_heads(rng, shape, head_dim):
    """FP32 array [..., head_dim] drawn from N(0,1) and normalised per head."""
    x = rng.standard_normal(size=tuple(shape) + (head_dim,), dtype=np.float32)
    x /= np.sqrt((x.astype(np.float64) ** 2).sum(axis=-1, keepdims=True)).astype(np.float32)
    return x


def gemv_bytes(n, k, m):
    """Algorithmic HBM bytes of one NVFP4 GEMV call: codes + scales + tensor scale + BF16 x + FP32 y."""
    return n * k // 2 + n * k // 16 + 4 + 2 * m * k + 4 * m * n


# The projection shapes of one synthetic 4B-shaped layer (d_model 3072, 32 q / 8 KV heads of 128, FFN 8192).
LAYER_SHAPES = {
    "qkv5120": (5120, 3072),
    "qkv6144": (6144, 3072),
    "qkvg10240": (10240, 3072),
    "gateup16384": (16384, 3072),
    "down": (3072, 8192),
    "o_proj": (3072, 4096),
    "square3072": (3072, 3072),
}

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
    """FP32 -> E4M3 codes, round to nearest even, |x| >= 448 saturating to 0x7e, NaN to 0x7f (with the sign).

    Below 2^-6 the result counts subnormal steps of 2^-9 (ties to even); above, the FP32 significand is rounded to
    3 bits (ties to even) and rebiased -- the same codes as the nearest-even table search, done on the bits."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> 24) & np.uint32(0x80)).astype(np.uint8)
    a = bits & np.uint32(0x7FFFFFFF)
    small = a < np.uint32(0x3C800000)
    # normal range (a >= 2^-6): round the significand to 3 bits, nearest even, rebias 127 -> 7
    code = (a >> 20) & np.uint32(1)
    code += a
    code += np.uint32(0x7FFFF)
    code >>= 20                                   # exponent (8 bits) and 3 significand bits
    code -= np.uint32(120 << 3)                   # rebias; wraps for small a, which is replaced below
    np.minimum(code, np.uint32(0x7E), out=code)
    if small.any():
        # subnormal range: steps of 2^-9, nearest even
        t = a[small].view(np.float32) * np.float32(512.0)
        lo = np.floor(t)
        half = t - lo
        steps = lo.astype(np.uint32)
        steps += (half > 0.5) | ((half == 0.5) & ((steps & np.uint32(1)) == 1))
        code[small] = steps
    code[a > np.uint32(0x7F800000)] = 0x7F          # NaN (above the saturation test, which NaN fails)
    out = code.astype(np.uint8)
    out |= sign
    return out


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


# ------------------------------------------------------------------------------------- synthetic Dory model

MLP, SLIDING, FULL = 0, 1, 2

# The 4B-shaped decode configuration: d_model 3072, 32 q / 8 KV heads of 128, FFN 8192 (SwiGLU), 4 input / 40
# recurrent / 4 output sublayers alternating attention and MLP (24 + 24), one loop, every fourth attention
# sublayer global and the others sliding (window 1024 in a 1088-slot ring), vocab 131072 with an NVFP4 head.
DORY_4B = dict(hidden=3072, ffn=8192, heads=32, kv_heads=8, head_dim=128, vocab=131072, n_in=4, n_rec=40, n_out=4,
               loops=1, window=1024, ring_slots=1088, theta_sliding=1e6, theta_full=1e6)
# The real Dory 4B's shape (docs/dory.md:12-15 of the reference): hidden 2560, FFN 7168, 16 q / 4 KV heads of 256,
# 16 input / 40 recurrent / 16 output sublayers (9 of the 36 attention sublayers global), two loops, sliding window
# 1024 in the CPU session's ring of window + 16 slots (packs/dory/dory.cpp:43, 449), RoPE theta 1e4 sliding / 1e7
# global, FP8 caches in last_loop mode (the shipped card's defaults) and a BF16 LM head over 131072.
DORY_REAL = dict(hidden=2560, ffn=7168, heads=16, kv_heads=4, head_dim=256, vocab=131072, n_in=16, n_rec=40,
                 n_out=16, loops=2, window=1024, ring_slots=1040, theta_sliding=1e4, theta_full=1e7, kv_dtype=1,
                 kv_mode=1, bf16_head=True)
# A small model with the same structure for parity tests (two loops exercise the per-loop caches).
DORY_TINY = dict(hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64, vocab=1000, n_in=2, n_rec=4, n_out=2,
                 loops=2, window=48, ring_slots=64, theta_sliding=1e4, theta_full=1e6)


def dory_kinds(cfg):
    """Sublayer kinds: attention and MLP alternate (attention first); every fourth attention sublayer is global."""
    n = cfg["n_in"] + cfg["n_rec"] + cfg["n_out"]
    kinds, a = [], 0
    for l in range(n):
        if l % 2 == 0:
            kinds.append(FULL if a % 4 == 3 else SLIDING)
            a += 1
        else:
            kinds.append(MLP)
    return kinds


class DoryWeights:
    """Random-init weights of a Dory-shaped model with the scale vectors already folded (as the reference's model
    constructor leaves them): NVFP4 projections with the benchmark distributions (uniform codes, |N(0,1)|*0.05
    scales); qscale, gscale ~ U(0.5, 1.5); sg, su ~ U(5, 15) (so silu sees arguments of order one);
    lr ~ U(0.02, 0.1); logit_scale ~ U(0.5, 1.5)."""

    def __init__(self, cfg, seed=0, context=4096, workers=8):
        import concurrent.futures
        self.cfg = dict(cfg)
        self.cfg["context"] = int(context)
        H, F = cfg["hidden"], cfg["ffn"]
        Q, KV = cfg["heads"] * cfg["head_dim"], cfg["kv_heads"] * cfg["head_dim"]
        self.kinds = dory_kinds(cfg)

        def layer(i):   # every sublayer (and the head, i = len) draws from its own stream of the seed
            rng = np.random.default_rng([seed, i])
            if i == len(self.kinds):
                if cfg.get("bf16_head"):   # a BF16 head as a checkpoint's lm_head.weight: N(0,1) rounded to BF16
                    w = f32_to_bf16(rng.standard_normal((cfg["vocab"], H), dtype=np.float32))
                    return w, rng.uniform(0.5, 1.5, cfg["vocab"]).astype(np.float32)
                return nvfp4_weight(rng, cfg["vocab"], H), rng.uniform(0.5, 1.5, cfg["vocab"]).astype(np.float32)
            kind = self.kinds[i]
            L = {"kind": kind, "lr": rng.uniform(0.02, 0.1, H).astype(np.float32)}
            if kind == MLP:
                L["gate"] = nvfp4_weight(rng, F, H)
                L["up"] = nvfp4_weight(rng, F, H)
                L["down"] = nvfp4_weight(rng, H, F)
                L["sg"] = rng.uniform(5, 15, F).astype(np.float32)
                L["su"] = rng.uniform(5, 15, F).astype(np.float32)
            else:
                for name, n in (("q", Q), ("k", KV), ("v", KV), ("g", Q)):
                    L[name] = nvfp4_weight(rng, n, H)
                L["o"] = nvfp4_weight(rng, H, Q)
                L["qscale"] = rng.uniform(0.5, 1.5, Q).astype(np.float32)
                L["gscale"] = rng.uniform(0.5, 1.5, Q).astype(np.float32)
            return L

        with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as ex:
            parts = list(ex.map(layer, range(len(self.kinds) + 1)))
        self.layers = parts[:-1]
        self.head, self.logit_scale = parts[-1]
        self.head_bf16 = None
        if cfg.get("bf16_head"):
            self.head_bf16, self.head = self.head, None

    def n_attn(self):
        return sum(1 for k in self.kinds if k != MLP)

    def weight_bytes(self):
        b = self.head[0].nbytes + self.head[1].nbytes if self.head is not None else self.head_bf16.nbytes
        for L in self.layers:
            for name in ("q", "k", "v", "g", "o", "gate", "up", "down"):
                if name in L:
                    b += L[name][0].nbytes + L[name][1].nbytes
        return b


def dory_structs(w, nvfp4_type, layer_type, config_type):
    """ctypes views (config, layer array, head) of DoryWeights for a C ABI with the xtg_dory_* layouts."""
    def nv(t):
        codes, scales, glob = t
        return nvfp4_type(codes.ctypes.data, scales.ctypes.data, glob, codes.shape[0], codes.shape[1] * 2)

    zero = nvfp4_type(None, None, 1.0, 0, 0)
    arr = (layer_type * len(w.layers))()
    for i, L in enumerate(w.layers):
        s = layer_type()
        s.kind = L["kind"]
        for name in ("q", "k", "v", "g", "o", "gate", "up", "down"):
            setattr(s, name, nv(L[name]) if name in L else zero)
        for name in ("qscale", "gscale", "sg", "su", "lr"):
            setattr(s, name, L[name].ctypes.data if name in L else None)
        arr[i] = s
    c = w.cfg
    cfg = config_type(c["hidden"], c["ffn"], c["heads"], c["kv_heads"], c["head_dim"], c["vocab"], c["n_in"],
                      c["n_rec"], c["n_out"], c["loops"], c["window"], c["ring_slots"], c["context"],
                      c["theta_sliding"], c["theta_full"], c.get("kv_dtype", 0), c.get("kv_mode", 0))
    return cfg, arr, nv(w.head) if w.head is not None else zero


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

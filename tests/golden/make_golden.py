"""Writes the golden vectors in this directory from the reference engine's own CPU kernels.

The reference (engine/src/{fp,kernels,kv}.cpp) is compiled from its sources by oracle/Makefile into
oracle/_ref/libxtgref.so (`make -C oracle ref`, needs the reference tree). This script feeds that library
seeded inputs and stores inputs and outputs as .npz (no pickles). The vectors pin the oracle restatement on
machines without the reference tree. Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, ROOT)

import oracle as orc  # noqa: E402


def load_workloads():
    import importlib.util
    spec = importlib.util.spec_from_file_location("wl", os.path.join(ROOT, "xtier-go_amd", "workloads.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


wl = load_workloads()


def nvfp4_cases():
    rng = np.random.default_rng(20261201)
    # kernels_test.cpp:57-87 shapes: two fused weights over k = 256, m = 1, 2, 7
    for m in (1, 2, 7):
        a = (rng.integers(0, 256, (70, 128), dtype=np.uint8), (0x20 + rng.integers(0, 0x30, (70, 16))).astype(np.uint8), 0.37)
        b = (rng.integers(0, 256, (33, 128), dtype=np.uint8), (0x20 + rng.integers(0, 0x30, (33, 16))).astype(np.uint8), 0.37)
        x = rng.uniform(-1, 1, (m, 256)).astype(np.float32)
        yield "nvfp4_kt_m%d" % m, [a, b], x
    # the benchmark distributions (uniform codes, |N(0,1)|*0.05 scales) at k = 1024 (unit BF16 rows), m = 1 and 8
    for m in (1, 8):
        w = wl.nvfp4_weight(rng, 64, 1024)
        x = wl.bf16_to_f32(wl.unit_rows_bf16(rng, m, 1024))
        yield "nvfp4_cfg_m%d" % m, [w], x


def attention_cases():
    rng = np.random.default_rng(20261202)
    # kernels_test.cpp:139-141 cases with the cached lengths cut to keep the files small
    heads, kvh, d = 8, 2, 64
    for cached, n_q, window, fp8 in ((300, 1, 0, 0), (700, 1, 0, 0), (300, 1, 64, 0), (100, 37, 0, 0),
                                     (100, 37, 16, 1), (0, 20, 0, 1), (400, 3, 128, 1)):
        yield ("attn_kt_c%d_q%d_w%d_%s" % (cached, n_q, window, "fp8" if fp8 else "bf16"), heads, kvh, d, cached, n_q,
               window, fp8, 0.7, rng)
    # the decode head layout (32 q / 8 KV heads of 128) at a short context, BF16, n_q 1 and 8
    for n_q in (1, 8):
        yield "attn_cfg_c320_q%d" % n_q, 32, 8, 128, 320, n_q, 0, 0, None, rng


def write_attention(name, heads, kvh, d, cached, n_q, window, fp8, scale, rng):
    total = cached + n_q
    K = rng.uniform(-1, 1, (total, kvh, d)).astype(np.float32)
    V = rng.uniform(-1, 1, (total, kvh, d)).astype(np.float32)
    q = rng.uniform(-1, 1, (n_q, heads, d)).astype(np.float32)
    if not fp8:   # BF16 caches: cached rows BF16-exact, kept as 16-bit words in the file
        K[:cached] = wl.bf16_to_f32(wl.f32_to_bf16(K[:cached]))
        V[:cached] = wl.bf16_to_f32(wl.f32_to_bf16(V[:cached]))
    slots = total + 8
    cache = orc.KvCache(kvh, d, slots, ring=window if window > 0 else 0, fp8=bool(fp8), use_ref=True)
    for p in range(0, cached, 50):
        n = min(50, cached - p)
        cache.store(p, K[p:p + n], V[p:p + n])
    out = orc.attention(q, K[cached:], V[cached:], cache, cached, heads, kvh, d, window=window, scale=scale,
                        pool_size=4)
    sc = np.float32(scale) if scale is not None else np.float32(1) / np.sqrt(np.float32(d))
    kv = {"K": K, "V": V} if fp8 else {"Kc": wl.f32_to_bf16(K[:cached]), "Vc": wl.f32_to_bf16(V[:cached]),
                                       "Kn": K[cached:], "Vn": V[cached:]}
    np.savez_compressed(os.path.join(HERE, name + ".npz"), q=q, cached=cached, window=window, fp8=fp8, scale=sc,
                        heads=heads, kv_heads=kvh, head_dim=d, pool_size=4, out=out, **kv)


def write_rows():
    rng = np.random.default_rng(20261203)
    r = orc.ref()
    x = rng.standard_normal((3, 3072)).astype(np.float32)
    b = rng.standard_normal((3, 3072)).astype(np.float32)
    lr = np.abs(rng.standard_normal(3072)).astype(np.float32) * 0.05
    qk = rng.standard_normal((2, 5, 128)).astype(np.float32)
    g = rng.standard_normal((2, 512)).astype(np.float32)
    u = rng.standard_normal((2, 512)).astype(np.float32)
    sg = rng.uniform(0.5, 1.5, 512).astype(np.float32)
    su = rng.uniform(0.5, 1.5, 512).astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "rows.npz"), x=x, b=b, lr=lr, qk=qk, g=g, u=u, sg=sg, su=su,
                        justnorm=orc.justnorm(x, use_ref=True), slerp=orc.slerp_residual(x, b, lr, use_ref=True),
                        rope=orc.rope(qk, 5, 128, 40000, 1e6, use_ref=True),
                        swiglu=orc.swiglu_scaled(g, u, sg, su, use_ref=True))
    del r


def write_bf16():
    """matmul_bf16 (kernels.cpp:140-155): random BF16 weights (N(0,1) rounded to nearest even) and FP32 rows, at
    k = 320 (not a multiple of the 128-wide tiles) and k = 260 (k % 8 == 4, the smallest granule the reference's
    GPU path takes), m = 1, 3, 8."""
    rng = np.random.default_rng(20261204)
    for k in (320, 260):
        w = wl.f32_to_bf16(rng.standard_normal((96, k)).astype(np.float32))
        arrays = {"w": w}
        for m in (1, 3, 8):
            x = rng.uniform(-1, 1, (m, k)).astype(np.float32)
            arrays["x%d" % m] = x
            arrays["y%d" % m] = orc.matmul_bf16(w, x, threads=4, use_ref=True)
        np.savez_compressed(os.path.join(HERE, "bf16_k%d.npz" % k), **arrays)


# The Dory composition against the reference pack's own CPU session (packs/dory/dory.cpp:304-578, compiled into
# oracle/_ref): a synthetic checkpoint written by tests/make_checkpoint.py (deterministic for a seed and variant; its
# sha256 is kept with the vectors), driven through Session::forward with a schedule of calls. Each schedule entry is
# (pos0, token offset, n): the session is rewound to pos0 when it stands elsewhere (speculative decoding's rewind,
# dory.cpp:580-589), then forwards tokens[off:off + n] with logits for every row.
DORY_SCHEDULE = ([(0, 0, 30)] +                                       # a prompt in one chunk
                 [(p, p, 8) for p in range(30, 62, 8)] +              # 8-row verify steps
                 [(p, p, 1) for p in range(62, 90)] +                 # single steps past the 64-slot ring's wrap
                 [(90, 100, 8), (93, 93, 1)] +                        # 8 drafts, 3 accepted: rewind to 93
                 [(p, p, 1) for p in range(94, 100)])
DORY_TOKENS = 108
# (name, checkpoint variant, seed, launch options); the options are the pack's (dory.cpp:136-170)
DORY_CASES = [
    ("tiny_bf16_per_loop", "tiny", 3, {"kv_dtype": "bf16", "kv_mode": "per_loop"}),
    ("tiny_fp8_per_loop", "tiny", 3, {"kv_dtype": "fp8", "kv_mode": "per_loop"}),
    ("tiny_bf16_last_loop", "tiny", 3, {"kv_dtype": "bf16", "kv_mode": "last_loop"}),
    ("tiny_fp8_last_loop", "tiny", 3, {"kv_dtype": "fp8", "kv_mode": "last_loop"}),
    ("tiny_fp8_loops1", "tiny", 3, {"kv_dtype": "fp8", "kv_mode": "per_loop", "loops": 1}),
    ("d256_fp8_last_loop", "d256", 5, {"kv_dtype": "fp8"}),   # the checkpoint's (and the shipped card's) defaults
    ("d256_bf16_per_loop", "d256", 5, {"kv_dtype": "bf16", "kv_mode": "per_loop"}),
]


def checkpoint(variant, seed, root="/tmp/xtg_golden_ckpt"):
    import hashlib
    import subprocess
    d = os.path.join(root, "%s_%d" % (variant, seed))
    if not os.path.exists(os.path.join(d, "model.safetensors")):
        subprocess.run([sys.executable, os.path.join(ROOT, "tests", "make_checkpoint.py"), d, str(seed), variant],
                       check=True)
    with open(os.path.join(d, "model.safetensors"), "rb") as f:
        return d, hashlib.sha256(f.read()).hexdigest()


def write_dory():
    """Logits of the reference's DorySession over DORY_SCHEDULE for each case: a third of the rows as they are, and
    for every row its argmax, sum and sum of squares (float64)."""
    import json
    for name, variant, seed, opts in DORY_CASES:
        d, sha = checkpoint(variant, seed)
        options = dict({"backend": "cpu", "context": 256}, **opts)
        r = orc.RefDory(d, options, threads=4)
        tokens = np.random.default_rng(seed * 1000 + 7).integers(0, r.vocab, DORY_TOKENS).astype(np.int32)
        rows = []
        for pos0, off, n in DORY_SCHEDULE:
            if r.n_past != pos0:
                assert r.rewind(pos0), (name, pos0)
            rows.append(r.forward(tokens[off:off + n]))
        r.close()
        logits = np.concatenate(rows).astype(np.float32)
        keep = np.arange(0, len(logits), 3)
        l64 = logits.astype(np.float64)
        np.savez_compressed(os.path.join(HERE, "dory_%s.npz" % name), variant=variant, seed=seed, sha256=sha,
                            options=json.dumps(options), schedule=np.array(DORY_SCHEDULE, np.int64),
                            tokens=tokens, rows=keep, logits=logits[keep], argmax=logits.argmax(1),
                            sums=l64.sum(1), sumsq=(l64 * l64).sum(1))


def main():
    if not orc.ref_available():
        sys.exit("oracle/_ref/libxtgref.so is missing: run `make -C oracle ref` where the reference tree exists")
    only = set(sys.argv[1:])   # e.g. "bf16": write that group only
    if only:
        if "bf16" in only:
            write_bf16()
        if "dory" in only:
            write_dory()
        print("golden vectors written to", HERE)
        return
    write_bf16()
    for name, ws, x in nvfp4_cases():
        ys = orc.matmul_nvfp4(ws, x, use_ref=True, threads=4)
        arrays = {"x": x}
        for i, (c, s, g) in enumerate(ws):
            arrays["codes%d" % i] = c
            arrays["scales%d" % i] = s
            arrays["glob%d" % i] = np.float32(g)
            arrays["y%d" % i] = ys[i]
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
    for case in attention_cases():
        write_attention(*case)
    write_rows()
    write_dory()
    print("golden vectors written to", HERE)


if __name__ == "__main__":
    main()

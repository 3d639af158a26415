"""A seeded random sweep against the oracle, past the fixed cases of the other tests: NVFP4 projections of random
shapes (1-4 weights sharing K, N up to 3000, K up to 5104, 1-8 rows on the GEMV and 9-64 on the GEMM, FP32 or BF16
rows), the attention call over random cached lengths, row counts, windows, rings and head layouts (BF16 and FP8
caches), and sampling with random filters over rows of 5 to 131072 logits. Bars as elsewhere: rel-L2 <= 1e-5 against
the oracle; sampled tokens equal unless the oracle's draw lies within 1e-6 of a running-sum boundary."""
import numpy as np
import pytest

from test_gpu_attention import rel_l2, run_case

CASES = 300


@pytest.mark.gpu
def test_random_sweep(hip, pkg, orc, wl):
    rng = np.random.default_rng(20261202)
    fails = []
    for case in range(CASES):
        kind = case % 3
        if kind == 0:   # projections
            nw = int(rng.integers(1, 5))
            k = 16 * int(rng.integers(1, 320))
            ns = [int(rng.integers(1, 3000)) for _ in range(nw)]
            m = int(rng.integers(1, 9)) if rng.random() < 0.8 else int(rng.integers(9, 65))
            bf16 = bool(rng.integers(0, 2))
            ws = [pkg.Weight(*wl.nvfp4_weight(rng, n, k)) for n in ns]
            x = rng.standard_normal((m, k)).astype(np.float32)
            if bf16:
                xb = wl.f32_to_bf16(x)
                x = wl.bf16_to_f32(xb).astype(np.float32)
                dx = hip.array(xb)
            else:
                dx = hip.array(x)
            dy = hip.array(shape=(m * sum(ns),))
            hip.matmul_dev(ws, dx, pkg.X_BF16 if bf16 else pkg.X_F32, m, dy)
            got = dy.numpy()
            ref = orc.matmul_nvfp4([(w.codes, w.scales, w.glob) for w in ws], x)
            off = 0
            for i, n in enumerate(ns):
                e = rel_l2(got[off:off + m * n].reshape(m, n), ref[i])
                off += m * n
                if not e <= 1e-5:
                    fails.append(("matmul", k, ns, m, bf16, i, e))
            dx.free()
            dy.free()
            for w in ws:
                hip.release_weight(w)
        elif kind == 1:   # attention
            heads, kvh, d = [(8, 2, 64), (4, 1, 64), (16, 2, 128), (32, 8, 128), (8, 8, 64)][int(rng.integers(0, 5))]
            cached, n_q = int(rng.integers(0, 2500)), int(rng.integers(1, 40))
            window = 0 if rng.random() < 0.5 else int(rng.integers(1, 400))
            fp8 = bool(rng.random() < 0.3)
            ring = window + int(rng.integers(n_q, n_q + 64)) if window > 0 and rng.random() < 0.5 else None
            out, ref, _ = run_case(hip, orc, cached, n_q, window, heads, kvh, d, None, rng, ring=ring, fp8=fp8)
            e = rel_l2(out, ref)
            if not e <= 1e-5:
                fails.append(("attention", heads, kvh, d, cached, n_q, window, ring, fp8, e))
        else:   # sampling
            rows, n = int(rng.integers(1, 9)), int(rng.choice([5, 300, 2048, 4097, 70000, 131072]))
            x = (rng.standard_normal((rows, n)) * rng.choice([0.3, 1, 4])).astype(np.float32)
            p = dict(temperature=float(rng.choice([0.0, 0.5, 1.0, 1.7])), top_p=float(rng.choice([1.0, 0.95, 0.6, 0.1])),
                     top_k=int(rng.choice([0, 1, 3, 50, 500, 5000])), min_p=float(rng.choice([0.0, 0.02, 0.3])))
            u = rng.random(rows)
            dx, dout = hip.array(x), hip.array(shape=(8,), dtype=np.int32)
            hip.sample(dx, rows, n, u, dout, **p)
            got = dout.numpy()[:rows]
            dx.free()
            dout.free()
            want, margin = orc.sample(x, u, **p)
            for r in range(rows):
                if got[r] != want[r] and not margin[r] < 1e-6:
                    fails.append(("sample", rows, n, p, r, int(got[r]), int(want[r]), float(margin[r])))
    assert not fails, fails[:5]


@pytest.mark.gpu
def test_random_dory_configs(hip, orc, wl):
    """The decode-step composition over random small configurations -- widths, head layouts (4/2, 8/2, 2/1, 4/4,
    8/1 of 64, 128 or 256), windows of 8-48 in rings of 4-64 slots more (some too short to store before the scan),
    one or two loops, BF16 or FP8 caches, per_loop or last_loop KV mode -- through random calls: chunks of up to 40
    rows, then steps of 1-8. Every call's logits against the oracle's composition: rel-L2 <= 1e-3 and the same
    argmax per row."""
    rng = np.random.default_rng(20261203)
    fails = []
    for _ in range(40):
        heads, kvh = [(4, 2), (8, 2), (2, 1), (4, 4), (8, 1)][int(rng.integers(0, 5))]
        window = int(rng.choice([8, 16, 48]))
        cfg = dict(hidden=int(rng.choice([128, 256, 384])), ffn=int(rng.choice([256, 384, 512])), heads=heads,
                   kv_heads=kvh, head_dim=int(rng.choice([64, 128, 256])), vocab=int(rng.choice([500, 1000, 3000])),
                   n_in=2, n_rec=int(rng.choice([2, 4])), n_out=2, loops=int(rng.integers(1, 3)), window=window,
                   ring_slots=window + int(rng.choice([4, 16, 64])), theta_sliding=1e4, theta_full=1e6,
                   kv_dtype=int(rng.integers(0, 2)), kv_mode=int(rng.integers(0, 2)))
        context = 192
        w = wl.DoryWeights(cfg, seed=int(rng.integers(0, 1 << 30)), context=context)
        ref = orc.Dory(w, wl)
        dev = hip.dory(w)
        H, V = cfg["hidden"], cfg["vocab"]
        dx, dl = hip.array(shape=(64, H)), hip.array(shape=(64, V))
        pos = 0
        seq = [int(rng.integers(1, 41)) for _ in range(int(rng.integers(1, 4)))] + \
              [int(rng.integers(1, 9)) for _ in range(6)]
        for m in seq:
            x = rng.standard_normal((m, H)).astype(np.float32)
            x /= np.linalg.norm(x, axis=1, keepdims=True)
            dx.upload(np.concatenate([x, np.zeros((64 - m, H), np.float32)]))
            dev.forward(dx, m, pos, dl)
            got = dl.numpy()[:m]
            want = ref.forward(x, pos)
            e = float(np.linalg.norm(got.astype(np.float64) - want) / np.linalg.norm(want.astype(np.float64)))
            if not (e <= 1e-3 and (got.argmax(1) == want.argmax(1)).all()):
                fails.append((cfg, pos, m, e))
            pos += m
        dx.free()
        dl.free()
        dev.destroy()
    assert not fails, fails[:3]

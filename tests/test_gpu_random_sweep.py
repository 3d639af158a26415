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

#!/usr/bin/env python3
"""Benchmark of the NVFP4 skinny-GEMM hot path on one MI355X.

Workload (one step): the three projection shapes of one synthetic 4B-shaped layer -- QKV (N=5120, K=3072),
fused gate/up (2 x N=8192, K=3072, one launch) and down (N=3072, K=8192) -- each at M=1 (decode) and at M=8
(the speculative-verify batch): 6 calls of xtg_hip_matmul_nvfp4_dev on BF16 rows, each one GEMV launch that
builds its matrix-core operand from the rows itself. Weights follow the
benchmark distributions (uniform E2M1 codes, |N(0,1)|*0.05 E4M3 scales, tensor scale 1.0); activations are unit
BF16 rows. Consecutive calls read different copies of their weights, rotating over >= 1 GiB, so every launch
streams from HBM rather than from the 256 MB Infinity Cache. The steps are replayed from a HIP graph, so host launch
cost does not set the pace.

value: whole-step algorithmic bytes / device time per step (GB/s), inputs resident in HBM: the K timed steps are one
graph launch bracketed by HIP events on the backend's stream (host_ms_per_step: the wall clock of that launch through
the final synchronisation, host latency included).
roofline: the dominant kernel launch, the call (one GEMV launch: a kernel instantiation at one weight shape and row
count) that moves the most bytes of the step -- an instantiation can serve calls of different sizes (QKV and
gate/up at M=1 share one), and a roofline over a mixture of launch sizes describes none of them; by_kernel gives
the same figures grouped by instantiation. For each (shape, rows) a graph of one call per weight copy is replayed
between two HIP events on the backend's stream; achieved = the dominant call's algorithmic bytes per launch / its
launch time, against the 8 TB/s HBM peak (all_calls_*: the same over all 6 calls). traffic: that call's HBM bytes
per launch from rocprofv3 FETCH_SIZE / WRITE_SIZE passes over `bench.py --pmc-pass`, calibrated on a copy of known
size (profiles/gemv_layer_projections_traffic_pmc.md).
cpu_baseline: the reference engine's own CPU matmul_nvfp4 (oracle/_ref, compiled from the reference sources)
on the same shapes and inputs on this host's cores, or the oracle restatement when that library is absent.
"""
import argparse
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "xtier-go_amd")
HBM_PEAK_GBS = 8000.0
METRIC = "NVFP4 GEMV HBM GB/s (%peak) at M=1/8; synthetic 4B decode tok/s @4K/8K/32K"

# name, weights (n, k) fused in one call
SHAPES = [("qkv5120", [(5120, 3072)]), ("gateup2x8192", [(8192, 3072), (8192, 3072)]), ("down3072x8192", [(3072, 8192)])]
ROWS = (1, 8)


def load_package():
    if "xtier_go_amd" in sys.modules:
        return sys.modules["xtier_go_amd"]
    spec = importlib.util.spec_from_file_location("xtier_go_amd", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["xtier_go_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


# rocprofv3 sets ROCPROF_<domain>=1 in the environment of the program it traces. In a traced process the bench
# destroys no graph exec and captures graphs only for the 6-call step and the per-call GEMV launches: twice a traced
# run died (host SIGSEGV) inside hipGraphLaunch, both times after graph execs had been destroyed and new ones
# instantiated and replayed in the same process, and never without the tracer; the other sections run eagerly there.
TRACED = any(os.environ.get("ROCPROF_" + d) == "1" for d in (
    "KERNEL_TRACE", "HIP_RUNTIME_API_TRACE", "HIP_COMPILER_API_TRACE", "HSA_CORE_API_TRACE", "HSA_AMD_EXT_API_TRACE",
    "MEMORY_COPY_TRACE", "MEMORY_ALLOCATION_TRACE", "SCRATCH_MEMORY_TRACE"))


class Replay:
    """The launches fn() queues, replayable: captured into a HIP graph, or in a traced process (TRACED) fn itself
    run again on each replay. With profiling on, a graph replay is one entry under its label; eager launches are
    entries under their kernels' names (time() adds them up). keep_in_trace: the 6-call step's and the per-call
    GEMV graphs stay graphs in a traced process too (the configuration traced runs have replayed without failure: no
    graph exec is destroyed there before the process ends), so the trace times the launches the untraced run
    times."""

    def __init__(self, hip, label, fn, keep_in_trace=False):
        self.hip, self.label, self.fn, self.g = hip, label, fn, None
        self.keep = keep_in_trace and TRACED
        if not TRACED or self.keep:
            hip.graph_begin()
            fn()
            self.g = hip.graph_end(label)

    def launch(self):
        if self.g is not None:
            self.hip.graph_launch(self.g)
        else:
            self.fn()

    def time(self, rep, replays):
        """(ms, replays) of this replayable's launches in a profile report covering `replays` replays of it."""
        if self.g is not None:
            return rep[self.label]["ms"], rep[self.label]["calls"]
        return sum(v["ms"] for v in rep.values()), replays

    def destroy(self):
        if self.g is not None and not self.keep:   # a traced process destroys no graph exec before it ends
            self.hip.graph_destroy(self.g)
            self.g = None


def call_bytes(ws, m):
    """Algorithmic HBM bytes of one call: codes + scales + tensor scale per weight, BF16 x once, FP32 y."""
    k = ws[0][1]
    return sum(n * k // 2 + n * k // 16 + 4 for n, _ in ws) + 2 * m * k + 4 * m * sum(n for n, _ in ws)


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), for the CPU baseline rows."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(base, xs, seconds):
    """The reference's CPU matmul_nvfp4 (or the oracle) over the step's 6 calls, until `seconds` have passed, on
    all the host's threads; then the same on one thread for a quarter of that time."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    use_ref = orc.ref_available()
    ws_by = {name: [(w.codes, w.scales, w.glob) for w in base[name]] for name, _ in SHAPES}
    calls = [(name, m) for m in ROWS for name, _ in SHAPES]

    def run(threads, secs):
        orc.matmul_nvfp4(ws_by[calls[0][0]], xs[calls[0]], threads=threads, use_ref=use_ref)   # warm-up
        done, nbytes, t0 = 0, 0, time.perf_counter()
        while True:
            for name, m in calls:
                orc.matmul_nvfp4(ws_by[name], xs[(name, m)], threads=threads, use_ref=use_ref)
                nbytes += call_bytes(dict(SHAPES)[name], m)
            done += 1
            el = time.perf_counter() - t0
            if el >= secs:
                return nbytes / el / 1e9, done, el

    threads = os.cpu_count() or 1
    gbs, done, el = run(threads, seconds)
    gbs1, done1, el1 = run(1, seconds / 4)
    model = cpu_model()
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads,
            "kind": "reference" if use_ref else "port", "cpu": model,
            "sample": "%d passes over the step's 6 calls (QKV 5120, gate/up 2x8192, down 3072x8192 at M=1 and M=8, "
                      "same weights and inputs, one weight copy), %.1f s on %d threads of %s" % (done, el, threads,
                                                                                                 model),
            "single_thread": {"value": round(gbs1, 3), "unit": "GB/s", "cores": 1,
                              "sample": "%d passes, %.1f s on one thread" % (done1, el1)}}


# The NVFP4 GEMV workloads launch by launch: the 3072x3072 GEMV and the 4B layer's projections, including the QKV widths
# 6144 (32 q + 2 x 8 KV heads of 128) and 10240 (the fused q/k/v/g), at every verify batch size.
SWEEP = [("square3072", [(3072, 3072)]), ("qkv5120", [(5120, 3072)]), ("qkv6144", [(6144, 3072)]),
         ("qkvg10240", [(10240, 3072)]), ("gateup2x8192", [(8192, 3072), (8192, 3072)]),
         ("down3072x8192", [(3072, 8192)])]
SWEEP_ROWS = (1, 2, 4, 8)


def gemv_sweep(pkg, wl, hip, reps, cpu_seconds):
    """Per (shape, rows): a graph of one xtg_hip_matmul_nvfp4_dev call (one GEMV launch) per weight copy, the copies
    rotating over >= 1 GiB so each launch streams from HBM, replayed `reps` times between events on the backend's
    stream; per launch: microseconds, algorithmic GB/s (call_bytes) and the fraction of the HBM peak. The 3072x3072
    shape also on the CPU: the reference's matmul_nvfp4 on all threads and on one, on the same weights and row."""
    rng = np.random.default_rng(20261205)
    out = {}
    for name, shapes in SWEEP:
        base = [pkg.Weight(*wl.nvfp4_weight(rng, n, k)) for n, k in shapes]
        one = sum(w.codes.nbytes + w.scales.nbytes for w in base)
        copies = max(2, -(-(1 << 30) // one) + 1)
        sets = [[pkg.Weight(w.codes.copy(), w.scales.copy(), w.glob) for w in base] for _ in range(copies)]
        for ws in sets:
            for w in ws:
                hip.prepare(w)
        k = shapes[0][1]
        xb = wl.unit_rows_bf16(rng, 8, k)
        dx = hip.array(xb)
        dy = hip.array(shape=(8 * sum(n for n, _ in shapes) + 64,))
        for m in SWEEP_ROWS:
            hip.matmul_dev(sets[0], dx, pkg.X_BF16, m, dy)   # sizes what the call needs before the capture
            hip.finish()
            g = Replay(hip, "sweep_%s_m%d" % (name, m),
                       lambda: [hip.matmul_dev(ws, dx, pkg.X_BF16, m, dy) for ws in sets])
            g.launch()
            hip.finish()
            hip.profile(True)
            for _ in range(reps):
                g.launch()
            ms, n = g.time(hip.profile_report(), reps)
            hip.profile(False)
            g.destroy()
            us = ms * 1e3 / (n * copies)
            b = call_bytes(shapes, m)
            out["%s_m%d" % (name, m)] = {"us_per_launch": round(us, 3), "bytes": b, "gbs": round(b / us / 1e3, 1),
                                         "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
        log("GEMV sweep %-14s (%d copies): %s" % (name, copies, ", ".join(
            "M=%d %.2f us %.0f GB/s" % (m, out["%s_m%d" % (name, m)]["us_per_launch"], out["%s_m%d" % (name, m)]["gbs"])
            for m in SWEEP_ROWS)))
        if name == "square3072" and cpu_seconds > 0:
            sys.path.insert(0, os.path.join(ROOT, "oracle"))
            import oracle as orc
            use_ref = orc.ref_available()
            w = [(base[0].codes, base[0].scales, base[0].glob)]
            x = wl.bf16_to_f32(xb[:1])
            cpu = {}
            for threads, secs in ((os.cpu_count() or 1, cpu_seconds), (1, cpu_seconds)):
                orc.matmul_nvfp4(w, x, threads=threads, use_ref=use_ref)
                n, t0 = 0, time.perf_counter()
                while time.perf_counter() - t0 < secs:
                    orc.matmul_nvfp4(w, x, threads=threads, use_ref=use_ref)
                    n += 1
                el = (time.perf_counter() - t0) / n
                cpu["threads%d" % threads] = {"us": round(el * 1e6, 1), "gbs": round(call_bytes(shapes, 1) / el / 1e9, 3),
                                              "calls": n}
            cpu["kind"] = "reference" if use_ref else "port"
            cpu["cpu"] = cpu_model()
            out["square3072_cpu"] = cpu
            log("3072x3072 GEMV on the CPU (%s): %s" % (cpu["kind"], ", ".join(
                "%s %.1f us" % (kk, v["us"]) for kk, v in cpu.items() if kk.startswith("threads"))))
        dx.free()
        dy.free()
        for ws in sets:
            for w in ws:
                hip.release_weight(w)
        del sets
    return out


# Sizes of the read floor: the 6-call step's launches (QKV 5120, down 3072x8192, gate/up 2x8192 at M=8), a global
# layer's attention at 32K (BF16 K and V, 8 KV heads of 128) and the NVFP4 LM head (131072 x 3072).
READ_SIZES = [("qkv5120_m8", 9060352), ("down3072x8192_m8", 14385152), ("gateup2x8192_m8", 28885008),
              ("attention_ctx32768", 134217728), ("head131072x3072", 226492416)]
POOL_BYTES = 2 << 30


def read_floor(pkg, hip, reps):
    """The device's streaming-read roofline at the hot path's sizes (xtg_hip_read_probe, the reference's readsum
    probe): for each size, a graph of one read per slice of a 2 GiB pool (so every launch streams from HBM, not from
    the 256 MB Infinity Cache) replayed between events on the backend's stream; per launch us, GB/s and fraction of
    the 8 TB/s peak."""
    pool = hip.alloc(POOL_BYTES)
    out = {}
    for name, size in READ_SIZES:
        size = size // 16 * 16
        copies = max(2, POOL_BYTES // size)
        parts = hip.array(shape=(copies * hip.read_probe_partials(size),), dtype=np.uint32)
        per = hip.read_probe_partials(size) * 4

        def reads():
            for c in range(copies):
                hip.read_probe(pool + c * size, size, parts.ptr + c * per)

        g = Replay(hip, "read_%s" % name, reads)
        g.launch()
        hip.finish()
        hip.profile(True)
        for _ in range(reps):
            g.launch()
        ms, n = g.time(hip.profile_report(), reps)
        hip.profile(False)
        g.destroy()
        parts.free()
        us = ms * 1e3 / (n * copies)
        out[name] = {"bytes": size, "us": round(us, 3), "gbs": round(size / us / 1e3, 1),
                     "frac": round(size / us / 1e3 / HBM_PEAK_GBS, 4), "copies": copies}
        log("read floor %-20s %10d B: %.2f us, %.0f GB/s (%.1f%% of HBM peak)"
            % (name, size, us, size / us / 1e3, size / us / 1e3 / HBM_PEAK_GBS * 100))
    hip.release(pool)
    return out


def decode_attention_bench(pkg, wl, hip, reps, cpu_seconds):
    """Decode attention over global caches and sliding rings through xtg_hip_attention (a call of one row block: its
    own keys and the scan in one launch, then the merge by heads; each launch between events on the backend's
    stream), 32 q / 8 KV heads of 128, unit-norm K / V / q:
    - global caches of 4K / 8K / 32K positions, 1 and 8 new rows at positions ctx ..;
    - a 1088-slot ring after 40000 decoded positions (slots hold 38912 .. 39999), window 1024, 1 and 8
      rows at 40000 ..; the q / k producer (RoPE, per-head norm, qscale) timed beside it (xtg_hip_qk_rope_norm).
    BF16 and FP8 caches. Each call reads one of `copies` caches with the same contents, rotating over >= 1 GiB so
    every call streams the cache from HBM. Algorithmic bytes: the visible K and V (ctx positions, or the whole ring)
    at 2 bytes (BF16) or 1 byte plus a 4-byte scale per (position, head) for each of K and V (FP8), plus q, the new k
    and v, and out in FP32; the roofline fraction is that over the scan launch's time (the launch that streams the
    cache: the scan, or the own keys and scan in one launch). The reference's CPU attention (oracle/_ref) on the
    same inputs beside it."""
    heads, kvh, d = 32, 8, 128
    rng = np.random.default_rng(61)
    out = {}
    cases = [("ctx%d" % c, c, 0, 0) for c in (4096, 8192, 32768)] + [("ring1088", 40000, 1088, 1024)]
    for fp8 in (False, True):
        for label, ctx, ring, window in cases:
            lo = ctx - ring if ring else 0
            n_pos = ctx - lo
            K = wl.unit_heads(rng, (n_pos, kvh), d)
            V = wl.unit_heads(rng, (n_pos, kvh), d)
            dK, dV = hip.array(K), hip.array(V)
            per_pos = kvh * (2 * d + (8 if fp8 else 0)) if fp8 else kvh * d * 4
            cache_bytes = (ring if ring else ctx) * per_pos
            copies = max(2, -(-(1 << 30) // cache_bytes) + 1)
            caches = []
            for _ in range(copies):
                c = hip.kv_cache(kvh, d, ctx + 8, ring=ring, dtype=1 if fp8 else 0)
                for p in range(0, n_pos, 8192):
                    n = min(8192, n_pos - p)
                    c.store(lo + p, n, dK.ptr + p * kvh * d * 4, dV.ptr + p * kvh * d * 4)
                caches.append(c)
            hip.finish()
            for n_q in (1, 8):
                q = wl.unit_heads(rng, (n_q, heads), d)
                kn = wl.unit_heads(rng, (n_q, kvh), d)
                vn = wl.unit_heads(rng, (n_q, kvh), d)
                dq, dk, dv, do = hip.array(q), hip.array(kn), hip.array(vn), hip.array(shape=(n_q, heads, d))
                qs = hip.array(rng.uniform(0.5, 1.5, heads * d).astype(np.float32))
                for c in caches[:2]:
                    hip.attention(c, dq, dk, dv, do, n_q, ctx, heads, window=window)
                hip.finish()
                hip.profile(True)
                for _ in range(reps):
                    for c in caches:
                        if ring:
                            hip.qk_rope_norm(dq, dk, n_q, heads, kvh, d, ctx, 1e6, qs)
                        hip.attention(c, dq, dk, dv, do, n_q, ctx, heads, window=window)
                rep = hip.profile_report()
                hip.profile(False)
                calls = reps * copies
                kern = {kk: round(v["ms"] * 1e3 / v["calls"], 3) for kk, v in rep.items()}
                scan = [kk for kk in rep if kk.startswith(("attn_scan_kernel", "attn_step_kernel"))][0]
                attn_us = sum(v["ms"] for kk, v in rep.items() if kk.startswith("attn_")) * 1e3 / calls
                visible = ring if ring else ctx
                b = visible * per_pos + 4 * d * (2 * heads * n_q + 2 * kvh * n_q)
                key = "%s_%s_q%d" % ("fp8" if fp8 else "bf16", label, n_q)
                out[key] = {"copies": copies, "bytes": b, "kernels_us": kern, "attention_us": round(attn_us, 3),
                            "scan_gbs": round(b / kern[scan] / 1e3, 1),
                            "frac": round(b / kern[scan] / 1e3 / HBM_PEAK_GBS, 4),
                            "call_gbs": round(b / attn_us / 1e3, 1)}
                log("attention %-4s %-9s n_q=%d: scan %.2f us (%.0f GB/s, %.1f%% of HBM peak), call %.2f us%s"
                    % ("FP8" if fp8 else "BF16", label, n_q, kern[scan], b / kern[scan] / 1e3,
                       b / kern[scan] / 1e3 / HBM_PEAK_GBS * 100, attn_us,
                       (", producer %.2f us" % kern["qk_rope_norm_kernel"]) if ring else ""))
                for a in (dq, dk, dv, do, qs):
                    a.free()
            for c in caches:
                c.destroy()
            dK.free()
            dV.free()
    if cpu_seconds > 0:
        out["cpu"] = cpu_attention(wl, rng, cpu_seconds)
    return out


def cpu_attention(wl, rng, seconds):
    """The reference's CPU attention (engine/src/kv.cpp:166-286, oracle/_ref; the oracle's restatement when that is
    absent) on the 4K global cache (1 and 8 rows) and the 1088-slot ring (8 rows), BF16 caches, on all threads and
    on one."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    use_ref = orc.ref_available()
    heads, kvh, d = 32, 8, 128
    out = {"kind": "reference" if use_ref else "port", "cpu": cpu_model()}
    per = seconds / 6
    for label, ctx, ring, window, n_q in (("ctx4096_q1", 4096, 0, 0, 1), ("ctx4096_q8", 4096, 0, 0, 8),
                                           ("ring1088_q8", 40000, 1088, 1024, 8)):
        lo = ctx - ring if ring else 0
        cache = orc.KvCache(kvh, d, ctx + 8, ring=ring, fp8=False, use_ref=use_ref)
        for p in range(lo, ctx, 1024):
            n = min(1024, ctx - p)
            cache.store(p, wl.unit_heads(rng, (n, kvh), d), wl.unit_heads(rng, (n, kvh), d))
        q = wl.unit_heads(rng, (n_q, heads), d)
        k, v = wl.unit_heads(rng, (n_q, kvh), d), wl.unit_heads(rng, (n_q, kvh), d)
        b = (ring if ring else ctx) * kvh * d * 4 + 4 * d * (2 * heads * n_q + 2 * kvh * n_q)
        for threads in (os.cpu_count() or 1, 1):
            orc.attention(q, k, v, cache, ctx, heads, kvh, d, window=window, pool_size=threads, threads=threads)
            n, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < per or n == 0:
                orc.attention(q, k, v, cache, ctx, heads, kvh, d, window=window, pool_size=threads, threads=threads)
                n += 1
            el = (time.perf_counter() - t0) / n
            out["%s_threads%d" % (label, threads)] = {"us": round(el * 1e6, 1), "gbs": round(b / el / 1e9, 3),
                                                      "calls": n}
        del cache
    log("attention on the CPU (%s): %s" % (out["kind"], ", ".join(
        "%s %.0f us" % (kk, v["us"]) for kk, v in out.items() if isinstance(v, dict))))
    return out


COPY_BYTES = 256 << 20


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_layer_projections_traffic_pmc.md")


def measured_traffic():
    """Per-call HBM bytes from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes over --pmc-pass (the JSON
    block of profiles/gemv_layer_projections_traffic_pmc.md, counters calibrated on a copy of known size), or
    None when that summary is absent."""
    try:
        text = open(TRAFFIC_FILE).read()
        block = text[text.index("```json") + 7:]
        return json.loads(block[:block.index("```")])["per_call"]
    except (OSError, ValueError, KeyError):
        return None


def pmc_pass(pkg, wl):
    """Counter pass: the copy first (known bytes read and written once), then the GEMV calls, each followed by a
    finish so dispatches stay apart, then 4 launches of the NVFP4 LM head. Kernel dispatch order: copy, one
    gemv_kernel per call (24), then prep_x_kernel + gemv_kernel per head launch."""
    hip = pkg.HipBackend(0)
    src, dst = hip.alloc(COPY_BYTES), hip.alloc(COPY_BYTES)
    hip.copy(src, dst, COPY_BYTES)
    hip.finish()
    rng = np.random.default_rng(20261201)
    base = {name: [pkg.Weight(*wl.nvfp4_weight(rng, n, k)) for n, k in shapes] for name, shapes in SHAPES}
    set_bytes = sum(w.codes.nbytes + w.scales.nbytes for ws in base.values() for w in ws)
    copies = max(2, -(-(1 << 30) // set_bytes) + 1)
    sets = []
    for _ in range(copies):
        s = {name: [pkg.Weight(w.codes.copy(), w.scales.copy(), w.glob) for w in ws] for name, ws in base.items()}
        for ws in s.values():
            for w in ws:
                hip.prepare(w)
        sets.append(s)
    dy = hip.array(shape=(8 * 16384 + 64,))
    i = 0
    for m in ROWS:
        for name, shapes in SHAPES:
            xb = wl.unit_rows_bf16(rng, m, shapes[0][1])
            dx = hip.array(xb)
            for _ in range(4):
                hip.matmul_dev(sets[i % copies][name], dx, pkg.X_BF16, m, dy)
                hip.finish()
                i += 1
            dx.free()
    for s in sets:
        for ws in s.values():
            for w in ws:
                hip.release_weight(w)
    # then the 4B-shaped model's NVFP4 LM head (131072 x 3072, one FP32 row prepared by prep_x_kernel), two weight
    # copies read in turn, 4 launches
    heads = [pkg.Weight(*wl.nvfp4_weight(rng, 131072, 3072)) for _ in range(2)]
    for w in heads:
        hip.prepare(w)
    x = rng.standard_normal((1, 3072)).astype(np.float32)
    dx = hip.array(x)
    dh = hip.array(shape=(131072,))
    for i in range(4):
        hip.matmul_dev([heads[i % 2]], dx, pkg.X_F32, 1, dh)
        hip.finish()
    hip.release(src)
    hip.release(dst)
    hip.close()


MFMA_F16_PEAK_TFLOPS = 2500.0   # MI355X dense f16 matrix-core peak


def prefill_gemm_bench(pkg, wl, hip, rows, reps):
    """The NVFP4 GEMM on a prefill chunk: one 4B-shaped layer's projections (q/k/v/g 10240x3072, fused gate/up
    2x8192x3072, o 3072x4096, down 3072x8192) at `rows` rows of FP32 activations, operand prepared once, each
    launch bracketed by events. Compute-bound: reported against the dense f16 matrix-core peak with the
    algorithmic 2 m n k flops (the default two-part operand issues twice that: each activation is a high and a low
    f16 part; with XTG_GEMM_PARTS=1 in the environment, the single-part operand issues them once)."""
    rng = np.random.default_rng(41)
    parts = 1 if os.environ.get("XTG_GEMM_PARTS") == "1" else 2   # matrix ops issued per useful one
    calls = [("qkvg10240", [(10240, 3072)]), ("gateup2x8192", [(8192, 3072), (8192, 3072)]),
             ("o3072x4096", [(3072, 4096)]), ("down3072x8192", [(3072, 8192)])]
    out = {"rows": rows, "per_call": {}}
    tot_flops, tot_us = 0.0, 0.0
    for name, shapes in calls:
        ws = [pkg.Weight(*wl.nvfp4_weight(rng, n, k)) for n, k in shapes]
        k = shapes[0][1]
        for w in ws:
            hip.prepare(w)
        x = rng.standard_normal((rows, k)).astype(np.float32)
        dx = hip.array(x)
        dy = hip.array(shape=(rows * sum(n for n, _ in shapes),))
        op = hip.array(shape=((rows + 7) // 8 * hip.x_operand_bytes(k),), dtype=np.uint8)
        hip.prep_x(dx, pkg.X_F32, rows, k, op)
        for _ in range(3):
            hip.matmul_op(ws, op, rows, dy)
        hip.finish()
        hip.profile(True)
        for _ in range(reps):
            hip.matmul_op(ws, op, rows, dy)
        rep = hip.profile_report()
        hip.profile(False)
        kname = [kk for kk in rep if kk.startswith("gemm_kernel")][0]
        us = rep[kname]["ms"] * 1e3 / rep[kname]["calls"]
        flops = 2.0 * rows * k * sum(n for n, _ in shapes)
        out["per_call"][name] = {"kernel": kname, "us_per_launch": round(us, 2),
                                 "tflops": round(flops / us / 1e6, 1),
                                 "frac": round(flops / us / 1e6 / MFMA_F16_PEAK_TFLOPS, 4)}
        tot_flops += flops
        tot_us += us
        log("prefill GEMM %s at %d rows: %s %.1f us, %.1f TFLOP/s (%.1f%% of the dense f16 peak; matrix-core "
            "issue %.1f%%)" % (name, rows, kname, us, flops / us / 1e6, flops / us / 1e6 / MFMA_F16_PEAK_TFLOPS * 100,
                               parts * flops / us / 1e6 / MFMA_F16_PEAK_TFLOPS * 100))
        for a in (dx, dy, op):
            a.free()
        for w in ws:
            hip.release_weight(w)
    achieved = tot_flops / tot_us / 1e6
    out["roofline"] = {"bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                       "unit": "TFLOP/s", "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4),
                       "issue_frac": round(parts * achieved / MFMA_F16_PEAK_TFLOPS, 4), "operand_parts": parts}
    return out


def prefill_attention_bench(pkg, wl, hip, rows, ctx, reps):
    """The attention ABI call on a prefill chunk of `rows` rows after `ctx` cached positions, on the 4B model's
    heads (32 query heads over 8 KV heads of 128, a BF16 global cache): the own-key, scan and merge launches,
    each bracketed by events. Reported as the algorithmic 4 d flops per (query head, visible key) pair."""
    rng = np.random.default_rng(43)
    heads, kvh, d = 32, 8, 128
    dc = hip.kv_cache(kvh, d, ctx + rows, ring=0)
    for p in range(0, ctx, 512):
        n = min(512, ctx - p)
        dc.store_host(p, wl.unit_heads(rng, (n, kvh), d), wl.unit_heads(rng, (n, kvh), d))
    dq = hip.array(wl.unit_heads(rng, (rows, heads), d))
    dk = hip.array(wl.unit_heads(rng, (rows, kvh), d))
    dv = hip.array(wl.unit_heads(rng, (rows, kvh), d))
    dout = hip.array(shape=(rows, heads, d))
    for _ in range(3):
        hip.attention(dc, dq, dk, dv, dout, rows, ctx, heads)
    hip.finish()
    hip.profile(True)
    for _ in range(reps):
        hip.attention(dc, dq, dk, dv, dout, rows, ctx, heads)
    rep = hip.profile_report()
    hip.profile(False)
    for a in (dq, dk, dv, dout):
        a.free()
    dc.destroy()
    us = sum(v["ms"] for v in rep.values()) * 1e3 / reps
    pairs = rows * heads * (ctx + (rows + 1) / 2.0)
    tflops = 4.0 * d * pairs / us / 1e6
    kern = {k: round(v["ms"] * 1e3 / v["calls"], 2) for k, v in rep.items()}
    log("prefill attention %d rows after %d cached: %.1f us per call (%s), %.1f TFLOP/s algorithmic"
        % (rows, ctx, us, ", ".join("%s %.1f us" % kv for kv in kern.items()), tflops))
    return {"rows": rows, "cached": ctx, "us_per_call": round(us, 2), "tflops": round(tflops, 1),
            "kernels_us": kern}


def bf16_head_bench(pkg, wl, hip, reps):
    """matmul_bf16 on the BF16 checkpoint's LM head shape (131072 x 2560, 671 MB): two copies (1.34 GB) read in
    turn so each launch streams from HBM; every launch bracketed by events on the backend's stream. Returns
    per-row-count kernel times and GB/s (algorithmic bytes: weights + FP32 x + FP32 y)."""
    n, k = 131072, 2560
    rng = np.random.default_rng(31)
    base = wl.f32_to_bf16(rng.standard_normal((n, k), dtype=np.float32))
    ws = [base, base.copy()]
    for w in ws:
        hip.prepare_bf16(w)
    x = rng.standard_normal((8, k)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    dx, dy = hip.array(x), hip.array(shape=(8, n))
    out = {"shape": [n, k]}
    for m in (1, 8):
        for w in ws:   # warm (and size the operand)
            hip.matmul_bf16_dev(w, dx, pkg.X_F32, m, dy)
        hip.finish()
        hip.profile(True)
        for _ in range(reps):
            for w in ws:
                hip.matmul_bf16_dev(w, dx, pkg.X_F32, m, dy)
        rep = hip.profile_report()
        hip.profile(False)
        name = [kk for kk in rep if kk.startswith("gemv_bf16_kernel")][0]
        us = rep[name]["ms"] * 1e3 / rep[name]["calls"]
        b = n * k * 2 + 4 * m * k + 4 * m * n
        out["m%d" % m] = {"kernel": name, "us_per_launch": round(us, 2), "bytes": b, "gbs": round(b / us / 1e3, 1),
                          "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
        log("BF16 head %dx%d M=%d: %s %.1f us, %.0f GB/s (%.1f%% of HBM peak)"
            % (n, k, m, name, us, b / us / 1e3, b / us / 1e3 / HBM_PEAK_GBS * 100))
    for w in ws:
        hip.release_bf16(w)
    dx.free()
    dy.free()
    return out


def sampling_bench(pkg, hip, reps):
    """The device sampler on 131072-wide logits (the vocabulary), 1 and 8 rows: greedy (argmax), temperature only
    (walk in index order), top_k 40, top_k 300 and top_p 0.9 (sorted candidates); events on the backend's stream
    around each call (its launches timed as one, under the name of the last: `kernel`)."""
    n = 131072
    rng = np.random.default_rng(51)
    x = (rng.standard_normal((8, n)) * 3).astype(np.float32)
    dx, dout = hip.array(x), hip.array(shape=(8,), dtype=np.int32)
    out = {"n": n}
    for label, p in (("greedy", dict(temperature=0.0)), ("temperature", dict(temperature=0.8)),
                     ("top_k40", dict(temperature=0.8, top_k=40)), ("top_k300", dict(temperature=0.8, top_k=300)),
                     ("top_p0.9", dict(temperature=0.8, top_p=0.9))):
        for m in (1, 8):
            u = rng.random(m)
            hip.sample(dx, m, n, u, dout, **p)
            hip.finish()
            hip.profile(True)
            for _ in range(reps):
                hip.sample(dx, m, n, u, dout, **p)
            rep = hip.profile_report()
            hip.profile(False)
            name = [kk for kk in rep if kk in ("sample_pick_kernel", "argmax_pick_kernel", "argmax_kernel")][0]
            us = rep[name]["ms"] * 1e3 / rep[name]["calls"]
            out["%s_m%d" % (label, m)] = {"kernel": name, "us": round(us, 2)}
            log("sampling %s, %d row(s) of %d logits: %s %.1f us" % (label, m, n, name, us))
    dx.free()
    dout.free()
    return out


def prefill_run(pkg, hip, dev, w, rng, prompts):
    """Prompt processing on the 4B-shaped model (BF16 caches): xtg_hip_dory_prefill over n unit-norm rows from
    position 0 in chunks of 512 with logits for the last row only (the reference's Logits::Last), queued eagerly;
    wall time from the call to the end of its work. Plus a per-kernel split (events around every launch) of the
    first prompt."""
    H, V = w.cfg["hidden"], w.cfg["vocab"]
    out = {}
    nmax = max(prompts)
    x = rng.standard_normal((nmax, H)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    dx, dl = hip.array(x), hip.array(shape=(1, V))
    dev.prefill(dx, 512, 0, pkg.LOGITS_LAST, dl)   # scratch sized, kernels loaded
    hip.finish()
    for n in prompts:
        times = []
        for _ in range(2):
            t = time.perf_counter()
            dev.prefill(dx, n, 0, pkg.LOGITS_LAST, dl)
            hip.finish()
            times.append(time.perf_counter() - t)
        s = min(times)
        out["prompt%d" % n] = {"s": round(s, 4), "tok_s": round(n / s, 1)}
        log("prefill %5d tokens (chunks of 512, last-row logits): %.1f ms, %.0f tok/s" % (n, s * 1e3, n / s))
    n = min(prompts)
    hip.profile(True)
    dev.prefill(dx, n, 0, pkg.LOGITS_LAST, dl)
    rep = hip.profile_report()
    hip.profile(False)
    tot = sum(v["ms"] for v in rep.values())
    out["kernels_prompt%d" % n] = {k: {"calls": v["calls"], "ms": round(v["ms"], 2)} for k, v in
                                   sorted(rep.items(), key=lambda kv: -kv[1]["ms"])}
    log("prefill %d tokens, kernel time %.1f ms: %s" % (n, tot, ", ".join(
        "%s %.1f" % (k, v["ms"]) for k, v in sorted(rep.items(), key=lambda kv: -kv[1]["ms"])[:6])))
    dx.free()
    dl.free()
    return out


def nvfp4_bytes(n, k):
    """Codes, E4M3 scales and the tensor scale of an n x k NVFP4 weight."""
    return n * k // 2 + n * k // 16 + 4


def attn_splits(c, ctx, ring, fp8=False):
    """The key splits the attention step's plan takes for one row (attn_plan in csrc/attention.hip: about 192
    work-groups, 512 on an FP8 cache by position, four waves of 32-slot tiles each, at least two tiles per wave on a
    cache by position and one on a ring)."""
    tiles = -(-ring // 32) if ring else -(-ctx // 32)
    mt = 1 if ring else 2
    want = max(1, (512 if fp8 and not ring else 192) // c["kv_heads"])
    return max(1, min(want, -(-tiles // (mt * 4)), tiles))


def decode_launches(w, wl, launches, ctx, fp8=False):
    """Per-launch algorithmic bytes and GB/s of one eager one-row step, from its launches in queue order (the fused
    one-token path: the input row's operand, then per attention sublayer the q/k/v/g projection, the attention step
    (producer and scan), the gate by heads and the o-projection, per MLP sublayer gate/up and down, then the head).
    Bytes per launch: the NVFP4 weights a projection streams plus its FP32 rows in and out; the attention step, the
    keys and values it must read (every position of a global cache, the window's of a ring) plus q / k / v in and its
    split partials out; the gate, those partials plus the gate rows in and the heads out."""
    c = w.cfg
    H, F, V = c["hidden"], c["ffn"], c["vocab"]
    d, kvh, heads = c["head_dim"], c["kv_heads"], c["heads"]
    Q, KV = heads * d, kvh * d
    per_key = kvh * ((2 * d + 8 + 4) if fp8 else (2 * d * 2 + 4))   # K, V (and FP8 scales), slot position
    roles = []   # (role, bytes) per launch
    li = 0
    seq = list(launches)
    i = 0

    def take(prefix):
        nonlocal i
        assert i < len(seq) and seq[i][0].startswith(prefix), (i, prefix, seq[i:i + 3])
        i += 1
        return seq[i - 1]

    def add(role, b):
        roles.append((role, b, seq[i - 1][0], seq[i - 1][1]))

    if seq and seq[0][0].startswith("prep_x"):
        take("prep_x")
        add("input operand", 4 * H * 2)
    for kind in w.kinds:
        if kind == wl.MLP:
            take("gemv")
            add("gate/up", 2 * nvfp4_bytes(F, H) + 4 * H * 4 + 4 * F)
            take("gemv")
            add("down", nvfp4_bytes(H, F) + 4 * F + 4 * H * 2)
            continue
        take("gemv")
        add("q/k/v/g", nvfp4_bytes(2 * Q + 2 * KV, H) + 4 * H * 4 + 4 * (2 * Q + 2 * KV))
        ring = c["ring_slots"] if kind == wl.SLIDING else 0
        visible = min(ctx, c["window"]) if ring else ctx
        part = (attn_splits(c, ctx, ring, fp8) + 1) * heads * (d + 2) * 4
        while i < len(seq) and not seq[i][0].startswith(("attn_gate", "gemv")):
            name = seq[i][0]
            take("")
            add("attention (global)" if not ring else "attention (ring)",
                visible * per_key + 4 * (Q + 2 * KV) + part if name.startswith("attn_step") else 0)
        take("attn_gate")
        add("gate", part + 4 * Q * 2)
        take("gemv")
        add("o", nvfp4_bytes(H, Q) + 4 * Q + 4 * H * 2)
    take("gemv")
    add("head", nvfp4_bytes(V, H) + 4 * H * 4 + 4 * V * 2)
    assert i == len(seq), seq[i:]
    out = {}
    for role, b, name, ms in roles:
        r = out.setdefault(role, {"launches": 0, "us": 0.0, "bytes": 0, "kernels": []})
        r["launches"] += 1
        r["us"] += ms * 1e3
        r["bytes"] += b
        if name not in r["kernels"]:
            r["kernels"].append(name)
    for r in out.values():
        r["us_per_launch"] = round(r["us"] / r["launches"], 3)
        r["bytes_per_launch"] = r["bytes"] // r["launches"]
        r["gbs"] = round(r["bytes"] / r["us"] / 1e3, 1) if r["us"] > 0 else None
        r["frac"] = round(r["bytes"] / r["us"] / 1e3 / HBM_PEAK_GBS, 4) if r["us"] > 0 else None
        r["us"] = round(r["us"], 1)
    return out


def decode_bench(pkg, wl, hip, contexts, reps, cpu_seconds, kv="both"):
    """The synthetic 4B-shaped looped-nGPT decode step (random-init NVFP4 weights, BF16 KV), one decode
    row (M=1) and one 8-row verify step per context, each captured as a HIP graph and replayed. The caches hold a
    synthetic context of unit-norm K / V rows; a replay re-decodes position ctx, so every replay is the same step."""
    ctx_max = max(contexts)
    t0 = time.perf_counter()
    w = wl.DoryWeights(wl.DORY_4B, seed=11, context=ctx_max + 64)
    log("decode: 4B-shaped model %.2f GB of NVFP4 weights generated in %.1f s" % (w.weight_bytes() / 1e9,
                                                                                time.perf_counter() - t0))
    t0 = time.perf_counter()
    dev = hip.dory(w)
    prep_s = time.perf_counter() - t0
    log("decode: weights prepared on the device in %.2f s (%.1f GB/s from host memory: copies of the checkpoint "
        "layout, repacked on the device)" % (prep_s, w.weight_bytes() / prep_s / 1e9))
    c = w.cfg
    kvh, d, ring, H, V = c["kv_heads"], c["head_dim"], c["ring_slots"], c["hidden"], c["vocab"]
    rng = np.random.default_rng(12)
    K = wl.unit_heads(rng, (ctx_max, kvh), d)
    Vv = wl.unit_heads(rng, (ctx_max, kvh), d)
    dK, dV = hip.array(K), hip.array(Vv)
    row = kvh * d * 4
    x = rng.standard_normal((8, H)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    dx = hip.array(x)
    dl = hip.array(shape=(8, V))
    attn = [a for a, k in enumerate(k for k in w.kinds if k != wl.MLP)]
    kinds = [k for k in w.kinds if k != wl.MLP]
    for a, kind in zip(attn, kinds):   # global caches: positions 0 .. ctx_max - 1 once
        if kind == wl.FULL:
            dev.cache(a).store(0, ctx_max, dK, dV)
    kv_step = {}
    results = {}
    for ctx in contexts:
        for a, kind in zip(attn, kinds):   # rings: the 1088 positions before ctx
            if kind == wl.SLIDING:
                dev.cache(a).store(ctx - ring, ring, dK.ptr + (ctx - ring) * row, dV.ptr + (ctx - ring) * row)
        hip.finish()
        n_full = kinds.count(wl.FULL)
        kv_step[ctx] = (n_full * ctx + (len(kinds) - n_full) * min(ring, c["window"])) * kvh * d * 2 * 2
        res = {}
        for m in (1, 8):
            dev.forward(dx, m, ctx, dl)   # eager once (scratch sized), then capture
            hip.finish()
            g = Replay(hip, "dory_step_ctx%d_m%d" % (ctx, m), lambda: dev.forward(dx, m, ctx, dl))
            for _ in range(3):
                g.launch()
            hip.finish()
            t = time.perf_counter()
            for _ in range(reps):
                g.launch()
            hip.finish()
            ms = (time.perf_counter() - t) / reps * 1e3
            g.destroy()
            step_bytes = w.weight_bytes() + kv_step[ctx]
            res["m%d" % m] = {"ms_per_step": round(ms, 4), "rows_per_s": round(m * 1e3 / ms, 1),
                              "hbm_gbs": round(step_bytes / (ms / 1e3) / 1e9, 1)}
        res["tok_s"] = res["m1"]["rows_per_s"]
        res["step_bytes_m1"] = w.weight_bytes() + kv_step[ctx]
        # one eager one-row step with every launch timed by events: per-launch bytes and GB/s by role
        dev.forward(dx, 1, ctx, dl)
        hip.finish()
        hip.profile(True, launches=True)
        dev.forward(dx, 1, ctx, dl)
        _, seq = hip.profile_report(launches=True)
        hip.profile(False)
        res["launches_m1"] = decode_launches(w, wl, seq, ctx)
        results["ctx%d" % ctx] = res
        log("decode ctx %5d: M=1 %.3f ms/token (%.0f tok/s, %.0f GB/s), M=8 verify %.3f ms/step (%.0f rows/s)"
            % (ctx, res["m1"]["ms_per_step"], res["tok_s"], res["m1"]["hbm_gbs"], res["m8"]["ms_per_step"],
               res["m8"]["rows_per_s"]))
        log("  eager step by launch: " + ", ".join(
            "%s %d x %.2f us %.0f GB/s" % (r, v["launches"], v["us_per_launch"], v["gbs"] or 0)
            for r, v in res["launches_m1"].items()))
    # per-kernel breakdown of one eager step at the largest context (events around every launch)
    hip.profile(True)
    dev.forward(dx, 1, ctx_max, dl)
    rep = hip.profile_report()
    hip.profile(False)
    kernels = {k: {"calls": v["calls"], "us": round(v["ms"] * 1e3, 1)} for k, v in
               sorted(rep.items(), key=lambda kv: -kv[1]["ms"])}
    results["kernels_ctx%d_m1_eager" % ctx_max] = kernels
    # the same model over FP8 caches (the reference Dory's default KV dtype): M=1 at every context
    fp8 = {} if kv != "bf16" else None
    import copy
    w8 = copy.copy(w)
    w8.cfg = dict(w.cfg, kv_dtype=1)
    dev8 = hip.dory(w8) if fp8 is not None else None
    for a, kind in zip(attn, kinds) if dev8 else []:
        if kind == wl.FULL:
            dev8.cache(a).store(0, ctx_max, dK, dV)
    for ctx in contexts if dev8 else []:
        for a, kind in zip(attn, kinds):
            if kind == wl.SLIDING:
                dev8.cache(a).store(ctx - ring, ring, dK.ptr + (ctx - ring) * row, dV.ptr + (ctx - ring) * row)
        hip.finish()
        dev8.forward(dx, 1, ctx, dl)
        hip.finish()
        g = Replay(hip, "dory_step_fp8_ctx%d" % ctx, lambda: dev8.forward(dx, 1, ctx, dl))
        for _ in range(3):
            g.launch()
        hip.finish()
        t = time.perf_counter()
        for _ in range(reps):
            g.launch()
        hip.finish()
        ms = (time.perf_counter() - t) / reps * 1e3
        g.destroy()
        kv8 = kv_step[ctx] // 2 + kv_step[ctx] // (2 * d) * 4   # 1-byte codes + a 4-byte scale per (row, head)
        fp8["ctx%d" % ctx] = {"ms_per_step": round(ms, 4), "tok_s": round(1e3 / ms, 1), "kv_bytes": kv8,
                              "hbm_gbs": round((w.weight_bytes() + kv8) / (ms / 1e3) / 1e9, 1)}
        hip.profile(True, launches=True)
        dev8.forward(dx, 1, ctx, dl)
        _, seq = hip.profile_report(launches=True)
        hip.profile(False)
        fp8["ctx%d" % ctx]["launches_m1"] = decode_launches(w8, wl, seq, ctx, fp8=True)
        log("decode ctx %5d, FP8 caches: M=1 %.3f ms/token (%.0f tok/s)" % (ctx, ms, 1e3 / ms))
    if dev8:
        # per-kernel breakdown of one eager FP8 step at the largest context (events around every launch)
        hip.profile(True)
        dev8.forward(dx, 1, ctx_max, dl)
        rep = hip.profile_report()
        hip.profile(False)
        results["kernels_fp8_ctx%d_m1_eager" % ctx_max] = {
            k: {"calls": v["calls"], "us": round(v["ms"] * 1e3, 1)} for k, v in
            sorted(rep.items(), key=lambda kv: -kv[1]["ms"])}
        dev8.destroy()
    results["fp8_kv_m1"] = fp8
    results["prepare"] = {"bytes": w.weight_bytes(), "s": round(prep_s, 3), "gbs": round(w.weight_bytes() / prep_s / 1e9, 2)}
    results["prefill"] = prefill_run(pkg, hip, dev, w, rng, [n for n in (4096, 32768) if n <= ctx_max])
    cpu = None
    if cpu_seconds > 0:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as orc
        ctx = min(contexts)
        ref = orc.Dory(w, wl)
        a_i = 0
        for a, kind in zip(attn, kinds):
            lo = 0 if kind == wl.FULL else ctx - ring
            ref.cache(a).store(lo, K[lo:ctx], Vv[lo:ctx])
        threads = os.cpu_count() or 1
        ref.forward(x[:1], ctx, threads=threads)
        n, t = 0, time.perf_counter()
        while time.perf_counter() - t < cpu_seconds or n == 0:
            ref.forward(x[:1], ctx, threads=threads)
            n += 1
        el = (time.perf_counter() - t) / n
        cpu = {"tok_s": round(1 / el, 3), "ms_per_token": round(el * 1e3, 2), "cores": threads, "kind": "port",
               "sample": "%d decode steps (M=1) of the oracle's composition at a %d context" % (n, ctx)}
        log("decode CPU (oracle, %d threads): %.2f tok/s at %d context" % (threads, cpu["tok_s"], ctx))
        del ref
    for a in (dK, dV, dx, dl):
        a.free()
    dev.destroy()
    results["cpu"] = cpu
    results["model"] = ("looped nGPT, d_model 3072, 32 q / 8 KV heads of 128, FFN 8192, 4/40/4 sublayers (24 attention: "
                        "6 global + 18 sliding 1024 in 1088-slot rings; 24 MLP), 1 loop, NVFP4 head over 131072")
    return results


def decode_eager_pass(pkg, wl, hip, ctx, kv_fp8, reps):
    """The decode step run eagerly (no graph capture), for a kernel trace of it: the 4B-shaped model over BF16 or
    FP8 caches holding a synthetic context of ctx unit-norm rows, `reps` one-row steps at position ctx, each
    launch on the backend's stream; prints the wall-clock milliseconds per step (launch overheads included)."""
    w = wl.DoryWeights(wl.DORY_4B, seed=11, context=ctx + 64)
    if kv_fp8:
        w.cfg = dict(w.cfg, kv_dtype=1)
    dev = hip.dory(w)
    c = w.cfg
    kvh, d, ring, H, V = c["kv_heads"], c["head_dim"], c["ring_slots"], c["hidden"], c["vocab"]
    rng = np.random.default_rng(12)
    dK, dV = hip.array(wl.unit_heads(rng, (ctx, kvh), d)), hip.array(wl.unit_heads(rng, (ctx, kvh), d))
    row = kvh * d * 4
    x = rng.standard_normal((1, H)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    dx, dl = hip.array(x), hip.array(shape=(1, V))
    kinds = [k for k in w.kinds if k != wl.MLP]
    for a, kind in enumerate(kinds):
        if kind == wl.FULL:
            dev.cache(a).store(0, ctx, dK, dV)
        else:
            dev.cache(a).store(ctx - ring, ring, dK.ptr + (ctx - ring) * row, dV.ptr + (ctx - ring) * row)
    dev.forward(dx, 1, ctx, dl)
    hip.finish()
    t = time.perf_counter()
    for _ in range(reps):
        dev.forward(dx, 1, ctx, dl)
    hip.finish()
    ms = (time.perf_counter() - t) / reps * 1e3
    log("eager decode step, %s caches, ctx %d: %.3f ms per step (wall clock, %d steps)"
        % ("FP8" if kv_fp8 else "BF16", ctx, ms, reps))
    for a in (dK, dV, dx, dl):
        a.free()
    dev.destroy()
    return ms


PHASES = ("entry", "loads issued", "first row load in", "operand built", "first weight tile in", "matrix ops done",
          "work-group barrier passed", "stores issued")


def gemv_phases(pkg, wl, reps):
    """Per-wave phase stamps of the step's 8-row GEMV launches (gemv_kernel on raw BF16 rows), from the phase-stamp
    build (xtier-go_amd/build.py --stamps, loaded through XTG_HIP_LIB): each wave records the constant-rate clock at
    its entry, once its loads are issued, when its first row load and its first weight tile have arrived, once its
    operand is built, after its matrix ops, after the work-group's barrier and after its stores. One launch at a
    time on weights not touched for >= 1 GiB of other calls (cold), events around it; times are from the first
    wave's entry (the earliest, median and latest wave to reach each point; medians over the repetitions)."""
    import ctypes
    setter = pkg.lib().xtg_hip_phase_stamps
    setter.restype = ctypes.c_int
    setter.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.POINTER(ctypes.c_int)]
    rng = np.random.default_rng(20261201)
    base = {name: [pkg.Weight(*wl.nvfp4_weight(rng, n, k)) for n, k in shapes] for name, shapes in SHAPES}
    set_bytes = sum(w.codes.nbytes + w.scales.nbytes for ws in base.values() for w in ws)
    copies = max(2, -(-(1 << 30) // set_bytes) + 1)
    hip = pkg.HipBackend(0)
    sets = []
    for _ in range(copies):
        s = {name: [pkg.Weight(w.codes.copy(), w.scales.copy(), w.glob) for w in ws] for name, ws in base.items()}
        for ws in s.values():
            for w in ws:
                hip.prepare(w)
        sets.append(s)
    dx = {name: hip.array(wl.unit_rows_bf16(rng, 8, shapes[0][1])) for name, shapes in SHAPES}
    dy = hip.array(shape=(8 * 16384 + 64,))
    records = 2 * 1024 * 16
    buf = hip.array(shape=(records, 8), dtype=np.uint64)
    zeros = np.zeros((records, 8), dtype=np.uint64)
    khz = ctypes.c_int(0)
    if setter(ctypes.c_void_p(buf.ptr), records, ctypes.byref(khz)) != 0 or khz.value <= 0:
        raise RuntimeError("xtg_hip_phase_stamps failed")
    per_us = khz.value / 1e3   # clock ticks per microsecond
    out = {"clock_mhz": khz.value / 1e3}
    calls = [(name, 8) for name, _ in SHAPES]
    for c in range(copies):   # every copy once, so each measured copy was last read >= 1 GiB of traffic ago
        for name, m in calls:
            hip.matmul_dev(sets[c][name], dx[name], pkg.X_BF16, m, dy)
    hip.finish()
    for i, (name, m) in enumerate(calls):
        rows = []
        launch_us = []
        kernel = None
        for r in range(reps):
            c = (r * len(calls) + i) % copies
            buf.upload(zeros)
            hip.profile(True)
            hip.matmul_dev(sets[c][name], dx[name], pkg.X_BF16, m, dy)
            rep = hip.profile_report()
            hip.profile(False)
            kernel, v = next((k, v) for k, v in rep.items() if k.startswith("gemv_kernel"))
            launch_us.append(v["ms"] * 1e3 / v["calls"])
            st = buf.numpy().astype(np.int64)
            st = st[st[:, 0] != 0]
            rows.append((st - st[:, :1].min()) / per_us)
        # stamp order in a record: entry, issued, operand, first weight, matrix done, barrier, stores, first row
        order = (0, 1, 7, 2, 3, 4, 5, 6)
        fast = np.median([[x[:, k].min() for k in order] for x in rows], axis=0)
        med = np.median([[np.median(x[:, k]) for k in order] for x in rows], axis=0)
        slow = np.median([[x[:, k].max() for k in order] for x in rows], axis=0)
        waves = int(np.median([x.shape[0] for x in rows]))
        key = "%s_m%d" % (name, m)
        out[key] = {"kernel": kernel, "waves": waves, "launch_us_events": round(float(np.median(launch_us)), 3),
                    "span_us": round(float(slow[-1]), 3),
                    "phases_us": {p: {"first": round(float(f), 3), "median": round(float(a), 3),
                                      "slowest": round(float(b), 3)} for p, f, a, b in zip(PHASES, fast, med, slow)}}
        log("%s (%s, %d waves): launch %.2f us by events, first entry to last store %.2f us"
            % (key, kernel, waves, out[key]["launch_us_events"], out[key]["span_us"]))
        for p, f, a, b in zip(PHASES, fast, med, slow):
            log("  %-26s first %6.2f  median %6.2f  slowest %6.2f us" % (p, f, a, b))
    setter(None, 0, ctypes.byref(khz))
    hip.close()
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=0, help="weight copies to rotate over (0: enough for 1 GiB)")
    ap.add_argument("--roofline-reps", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-contexts", default="4096,8192,32768")
    ap.add_argument("--decode-reps", type=int, default=50)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="the workload for a rocprofv3 --pmc pass: a 256 MiB device copy (the counters' calibration), "
                         "then each of the step's 6 calls 4 times on rotated weights; prints nothing else")
    ap.add_argument("--decode-kv", default="both", choices=["bf16", "both"],
                    help="KV dtypes of the decode measurement: the BF16 caches of the benchmark configuration only, "
                         "or also the FP8 caches of the reference Dory's default (M=1; the default)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the decode-step measurement (for profiling it); prints its own JSON line")
    ap.add_argument("--decode-eager", default="",
                    help="KV,CTX (e.g. fp8,4096): only the decode step run eagerly, without graph capture, for a "
                         "kernel trace of it (--decode-reps steps); prints its own JSON line")
    ap.add_argument("--read-floor", action="store_true",
                    help="only the streaming-read roofline at the hot path's sizes (for profiling it); prints its own "
                         "JSON line")
    ap.add_argument("--attention-only", action="store_true",
                    help="only the decode-attention calls through xtg_hip_attention (for profiling them); prints "
                         "its own JSON line")
    ap.add_argument("--sampling-only", action="store_true",
                    help="only the device sampler on 131072-wide logits (for profiling it); prints its own JSON line")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only the 6-call GEMV step and its roofline (for profiling them); the other sections are "
                         "left out of the JSON line")
    ap.add_argument("--gemv-phases", action="store_true",
                    help="only the per-wave phase stamps of the step's 8-row GEMV launches, from the phase-stamp "
                         "build (xtier-go_amd/build.py --stamps); prints its own JSON line")
    args = ap.parse_args()
    if args.gemv_phases:   # the phase-stamp build of the library, before the package loads one
        os.environ["XTG_HIP_LIB"] = os.path.join(PKG_DIR, "libxtg_hip_stamps.so")
        if not os.path.exists(os.environ["XTG_HIP_LIB"]):
            print("--gemv-phases needs the phase-stamp build: python xtier-go_amd/build.py --stamps", file=sys.stderr)
            sys.exit(2)
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the kernels are one GPU's share of a "
              "sharded layer); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    pkg = load_package()
    import xtier_go_amd.workloads as wl

    if args.pmc_pass:
        pmc_pass(pkg, wl)
        return

    if args.gemv_phases:
        ph = gemv_phases(pkg, wl, 5)
        print(json.dumps({"metric": "8-row GEMV launch phases (us from the first wave's entry)",
                          "value": ph["gateup2x8192_m8"]["span_us"], "unit": "us", "higher_is_better": False,
                          "gemv_phases": ph}))
        return

    if args.decode_eager:
        kvs, ctx = args.decode_eager.split(",")
        hip = pkg.HipBackend(0)
        ms = decode_eager_pass(pkg, wl, hip, int(ctx), kvs == "fp8", args.decode_reps)
        print(json.dumps({"metric": "eager decode step ms (%s caches, ctx %s)" % (kvs, ctx), "value": round(ms, 4),
                          "unit": "ms", "higher_is_better": False}))
        hip.close()
        return

    if args.attention_only:
        hip = pkg.HipBackend(0)
        att = decode_attention_bench(pkg, wl, hip, 3, 0)
        print(json.dumps({"metric": "decode attention call us (bf16 ring1088, one row)",
                          "value": att["bf16_ring1088_q1"]["attention_us"], "unit": "us", "higher_is_better": False,
                          "decode_attention": att}))
        hip.close()
        return

    if args.sampling_only:
        hip = pkg.HipBackend(0)
        samp = sampling_bench(pkg, hip, 20)
        print(json.dumps({"metric": "top_k 40 sampling call us (one row of 131072)",
                          "value": samp["top_k40_m1"]["us"], "unit": "us", "higher_is_better": False,
                          "sampling": samp}))
        hip.close()
        return

    if args.read_floor:
        hip = pkg.HipBackend(0)
        floor = read_floor(pkg, hip, 10)
        print(json.dumps({"metric": "streaming read GB/s", "value": floor["gateup2x8192_m8"]["gbs"], "unit": "GB/s",
                          "higher_is_better": True, "read_floor": floor}))
        hip.close()
        return

    if args.decode_only:
        hip = pkg.HipBackend(0)
        contexts = [int(v) for v in args.decode_contexts.split(",") if v]
        decode = decode_bench(pkg, wl, hip, contexts, args.decode_reps, 0 if args.no_cpu else args.cpu_seconds / 2,
                              args.decode_kv)
        first = "ctx%d" % contexts[0]
        print(json.dumps({"metric": "synthetic 4B decode tok/s", "value": decode[first]["tok_s"], "unit": "tok/s",
                          "n_gpus": 1, "higher_is_better": True, "data": "synthetic", "decode": decode}))
        hip.close()
        return

    rng = np.random.default_rng(20261201)
    base = {name: [pkg.Weight(*wl.nvfp4_weight(rng, n, k)) for n, k in shapes] for name, shapes in SHAPES}
    set_bytes = sum(w.codes.nbytes + w.scales.nbytes for ws in base.values() for w in ws)
    copies = args.copies or max(2, -(-(1 << 30) // set_bytes) + 1)
    log("weight set %.1f MB, %d copies (%.2f GiB)" % (set_bytes / 1e6, copies, copies * set_bytes / 2 ** 30))

    hip = pkg.HipBackend(0)
    info = hip.info()
    log("device %s, %d CUs" % (info["arch"], info["cus"]))
    sets = []
    for _ in range(copies):
        s = {name: [pkg.Weight(w.codes.copy(), w.scales.copy(), w.glob) for w in ws] for name, ws in base.items()}
        for ws in s.values():
            for w in ws:
                hip.prepare(w)
        sets.append(s)
    log("prepared %d weight copies (%.2f GB on the device)" % (copies, hip.info()["weight_bytes"] / 1e9))

    xs, dx = {}, {}
    for name, shapes in SHAPES:
        k = shapes[0][1]
        xb = wl.unit_rows_bf16(rng, 8, k)
        for m in ROWS:
            xs[(name, m)] = wl.bf16_to_f32(xb[:m])
            dx[(name, m)] = hip.array(xb[:m])
    dy = hip.array(shape=(8 * 16384 + 64,))
    calls = [(name, m) for m in ROWS for name, _ in SHAPES]
    step_bytes = sum(call_bytes(dict(SHAPES)[name], m) for name, m in calls)

    # The timed steps as one HIP graph: step s's call i reads weight copy (6 s + i) mod copies, so consecutive
    # launches stream different copies; the warm-up steps are a graph of their own, the same way.
    for name, m in calls:   # size the scratch before capturing
        hip.matmul_dev(sets[0][name], dx[(name, m)], pkg.X_BF16, m, dy)
    hip.finish()

    def steps(first, n):
        for st in range(first, first + n):
            for i, (name, m) in enumerate(calls):
                hip.matmul_dev(sets[(len(calls) * st + i) % copies][name], dx[(name, m)], pkg.X_BF16, m, dy)

    warm = Replay(hip, "warmup_steps", lambda: steps(0, max(1, args.warmup)), keep_in_trace=True)
    timed = Replay(hip, "timed_steps", lambda: steps(max(1, args.warmup), args.steps), keep_in_trace=True)
    warm.launch()
    hip.finish()
    # device time: events on the backend's stream around the one launch of the K steps (launch gaps between the
    # step's kernels included; host launch and synchronisation latency not); the wall clock of the same launch
    # through hip.finish() beside it. In a traced process (no graph) the steps run eagerly and the wall clock is
    # the figure.
    hip.profile(True)
    t0 = time.perf_counter()
    timed.launch()
    hip.finish()
    el_host = time.perf_counter() - t0
    el = timed.time(hip.profile_report(), 1)[0] / 1e3
    hip.profile(False)
    warm.destroy()
    timed.destroy()
    ms_per_step = el / args.steps * 1e3
    value = step_bytes / (el / args.steps) / 1e9
    log("timed %d steps: %.4f ms/step by device events (%.4f ms/step wall clock), %.1f GB/s whole-step (%.1f%% of "
        "HBM peak)" % (args.steps, ms_per_step, el_host / args.steps * 1e3, value, value / HBM_PEAK_GBS * 100))

    # roofline: per-call graphs (one GEMV launch per weight copy, the step's own kernel), timed by events
    per_call = {}
    gemv_graphs = {}
    for name, m in calls:
        gemv_graphs[(name, m)] = Replay(hip, "gemv_%s_m%d" % (name, m), lambda name=name, m=m: [
            hip.matmul_dev(sets[c][name], dx[(name, m)], pkg.X_BF16, m, dy) for c in range(copies)],
            keep_in_trace=True)
    for g in gemv_graphs.values():   # warm
        g.launch()
    hip.finish()
    timing = {}   # (ms, replays) per call: the calls' replays interleaved (graphs), or one call at a time (eager)
    if all(g.g is not None for g in gemv_graphs.values()):
        hip.profile(True)
        for _ in range(args.roofline_reps):
            for g in gemv_graphs.values():
                g.launch()
        rep = hip.profile_report()
        hip.profile(False)
        timing = {key: g.time(rep, args.roofline_reps) for key, g in gemv_graphs.items()}
    else:
        for key, g in gemv_graphs.items():
            hip.profile(True)
            for _ in range(args.roofline_reps):
                g.launch()
            timing[key] = g.time(hip.profile_report(), args.roofline_reps)
            hip.profile(False)
    for g in gemv_graphs.values():
        g.destroy()
    # the kernel that serves each call: one eager call each, named by the profile report
    kernel_of = {}
    for name, m in calls:
        hip.profile(True)
        hip.matmul_dev(sets[0][name], dx[(name, m)], pkg.X_BF16, m, dy)
        names = [k for k in hip.profile_report() if k.startswith(("gemv_kernel", "gemv_mx_kernel"))]
        hip.profile(False)
        kernel_of["%s_m%d" % (name, m)] = names[0]
    tot_bytes, tot_s = 0, 0.0
    by_kernel = {}
    for name, m in calls:
        ms, replays = timing[(name, m)]
        launches = replays * copies
        us = ms * 1e3 / launches
        b = call_bytes(dict(SHAPES)[name], m)
        key = "%s_m%d" % (name, m)
        per_call[key] = {"kernel": kernel_of[key], "us_per_launch": round(us, 3), "bytes": b,
                         "gbs": round(b / us / 1e3, 1), "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
        tot_bytes += b * launches
        tot_s += ms / 1e3
        kb = by_kernel.setdefault(kernel_of[key], {"bytes": 0.0, "s": 0.0, "calls": []})
        kb["bytes"] += b * launches
        kb["s"] += ms / 1e3
        kb["calls"].append(key)
    all_achieved = tot_bytes / tot_s / 1e9
    dom_call = max(per_call, key=lambda k: per_call[k]["bytes"])   # the launch that moves the most bytes
    dominant = per_call[dom_call]["kernel"]
    achieved = per_call[dom_call]["gbs"]
    traffic = measured_traffic()
    if traffic:
        for key, v in per_call.items():
            if key in traffic:
                v["traffic"] = traffic[key]["traffic_bytes"]
    by_m = {}
    for m in ROWS:
        keys = ["%s_m%d" % (name, m) for name, _ in SHAPES]
        by_m["m%d" % m] = round(sum(per_call[k]["bytes"] for k in keys) /
                                sum(per_call[k]["us_per_launch"] for k in keys) / 1e3, 1)
    log("GEMV: dominant launch %s (%s, %.0f%% of the step's bytes, %.0f%% of its kernel time) %.1f GB/s (%.1f%% "
        "of HBM peak); all 6 calls %.1f GB/s (%.1f%%); M=1 %.1f, M=8 %.1f GB/s"
        % (dominant, dom_call, 100 * per_call[dom_call]["bytes"] / step_bytes,
           100 * per_call[dom_call]["us_per_launch"] / sum(v["us_per_launch"] for v in per_call.values()), achieved,
           achieved / HBM_PEAK_GBS * 100, all_achieved, all_achieved / HBM_PEAK_GBS * 100, by_m["m1"], by_m["m8"]))
    for k, v in per_call.items():
        log("  %-22s %7.3f us  %7.1f GB/s" % (k, v["us_per_launch"], v["gbs"]))

    # the plain streaming read of each call's bytes (the same rotation over HBM): each call's time against it
    floor = read_floor(pkg, hip, 10)
    floor_by_bytes = sorted((v["bytes"], v["us"]) for v in floor.values())
    for key, v in per_call.items():
        near = min(floor_by_bytes, key=lambda bu: abs(bu[0] - v["bytes"]))
        if abs(near[0] - v["bytes"]) <= 0.05 * v["bytes"]:
            v["read_floor_us"] = near[1]
            v["of_read_floor"] = round(near[1] / v["us_per_launch"], 4)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(base, xs, args.cpu_seconds)
        log("CPU baseline (%s, %d threads): %.2f GB/s" % (cpu["kind"], cpu["cores"], cpu["value"]))

    sweep = attention = bf16_head = sampling = prefill = None
    if not args.gemv_only:
        sweep = gemv_sweep(pkg, wl, hip, 5, 0 if args.no_cpu else 1.0)
        attention = decode_attention_bench(pkg, wl, hip, 3, 0 if args.no_cpu else 6.0)
        bf16_head = bf16_head_bench(pkg, wl, hip, 10)
        sampling = sampling_bench(pkg, hip, 20)
        prefill = prefill_gemm_bench(pkg, wl, hip, 512, 10)
        # the single-part operand (XTG_GEMM_PARTS=1: f16 activations, half the matrix ops; not the default)
        os.environ["XTG_GEMM_PARTS"] = "1"
        try:
            prefill["single_part"] = {str(r): prefill_gemm_bench(pkg, wl, hip, r, 10) for r in (512, 2048)}
        finally:
            del os.environ["XTG_GEMM_PARTS"]
        prefill["rows2048"] = prefill_gemm_bench(pkg, wl, hip, 2048, 5)
        prefill["attention_ctx4096"] = prefill_attention_bench(pkg, wl, hip, 512, 4096, 10)

    decode = None
    if not args.no_decode and not args.gemv_only:
        for name in list(base):   # the projection bench's weights are no longer needed
            for s in sets:
                for w in s[name]:
                    hip.release_weight(w)
        sets.clear()
        contexts = [int(v) for v in args.decode_contexts.split(",") if v]
        decode = decode_bench(pkg, wl, hip, contexts, args.decode_reps, 0 if args.no_cpu else args.cpu_seconds / 2,
                              args.decode_kv)

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "host_ms_per_step": round(el_host / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "NVFP4 skinny GEMM over one 4B-shaped layer's projections: QKV N=5120 K=3072, fused gate/up "
                        "2x8192 K=3072, down N=3072 K=8192, each at M=1 and M=8 (6 calls per step, one GEMV launch "
                        "each that builds its operand from the rows; BF16 unit-row activations, FP32 out); weights "
                        "rotated over %d copies (%.2f GiB) so each "
                        "call reads HBM; the timed steps one HIP graph, timed by device events" % (copies, copies * set_bytes / 2 ** 30),
            "step_bytes": step_bytes,
            "gemv_gbs_by_rows": by_m,
            "per_call": per_call,
        },
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     # the dominant launch's HBM bytes (per-call values in config.per_call)
                     "traffic": per_call[dom_call].get("traffic"),
                     "kernel": dominant, "call": dom_call, "bytes_per_launch": per_call[dom_call]["bytes"],
                     "us_per_launch": per_call[dom_call]["us_per_launch"],
                     "byte_share": round(per_call[dom_call]["bytes"] / step_bytes, 4),
                     "by_kernel": {k: {"calls": v["calls"], "gbs": round(v["bytes"] / v["s"] / 1e9, 1),
                                       "frac": round(v["bytes"] / v["s"] / 1e9 / HBM_PEAK_GBS, 4),
                                       "byte_share": round(v["bytes"] / tot_bytes, 4)}
                                   for k, v in by_kernel.items()},
                     "all_calls_achieved": round(all_achieved, 1),
                     "all_calls_frac": round(all_achieved / HBM_PEAK_GBS, 4)},
        "cpu_baseline": cpu,
        "read_floor": floor,
        "gemv_sweep": sweep,
        "decode_attention": attention,
        "bf16_lm_head": bf16_head,
        "sampling": sampling,
        "prefill_gemm": prefill,
        "decode": decode,
    }
    hip.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

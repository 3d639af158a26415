"""ctypes binding of libxtg_hip.so, the gfx950 kernel layer behind include/xtg_hip.h.

The binding is a thin mirror of the C ABI for tests, benchmarks and Python callers. It has no CPU fallback:
when the library is not built, every call raises.
"""
import ctypes
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# XTG_HIP_LIB: another build of the same library (the phase-stamp build that `bench.py --gemv-phases` loads)
LIB_PATH = os.environ.get("XTG_HIP_LIB") or os.path.join(HERE, "libxtg_hip.so")

X_F32, X_BF16 = 0, 1
KV_BF16, KV_FP8 = 0, 1
LOGITS_NONE, LOGITS_LAST, LOGITS_ALL = 0, 1, 2   # xtg::Logits order (engine/include/xtg/model.h:28)

# Every function the header declares, with its ctypes signature: (name, restype, argtypes).
_P = ctypes.c_void_p
_I = ctypes.c_int
_SZ = ctypes.c_size_t
_ERR = [ctypes.c_char_p, _I]


class Nvfp4(ctypes.Structure):
    """xtg_nvfp4 (same fields as xtg::Nvfp4Weight, engine/include/xtg/kernels.h:13-20)."""
    _fields_ = [("codes", _P), ("scales", _P), ("glob", ctypes.c_float), ("n_out", _I), ("k", _I)]


class Bf16(ctypes.Structure):
    """xtg_bf16 (same fields as xtg::Bf16Weight, engine/include/xtg/kernels.h:22-25)."""
    _fields_ = [("data", _P), ("n_out", _I), ("k", _I)]


class Sampling(ctypes.Structure):
    """xtg_sampling (the fields of xtg::SamplingParams, engine/include/xtg/sampler.h:11-16)."""
    _fields_ = [("temperature", ctypes.c_float), ("top_p", ctypes.c_float), ("top_k", _I), ("min_p", ctypes.c_float)]


class AttnArgs(ctypes.Structure):
    """xtg_attn_args (the fields of xtg::AttnArgs, engine/include/xtg/kv.h:67-78)."""
    _fields_ = [("n_q", _I), ("pos0", ctypes.c_int64), ("heads", _I), ("kv_heads", _I), ("head_dim", _I),
                ("window", _I), ("scale", ctypes.c_float), ("q", _P), ("k", _P), ("v", _P), ("cache", _P),
                ("out", _P)]


_F = ctypes.c_float
_I64 = ctypes.c_int64


class DoryConfig(ctypes.Structure):
    """xtg_dory_config."""
    _fields_ = [(n, _I) for n in ("hidden", "ffn", "heads", "kv_heads", "head_dim", "vocab", "n_in", "n_rec", "n_out",
                                  "loops", "window", "ring_slots")] + \
               [("context", _I64), ("theta_sliding", _F), ("theta_full", _F), ("kv_dtype", _I), ("kv_mode", _I)]


class DoryLayer(ctypes.Structure):
    """xtg_dory_layer."""
    _fields_ = [("kind", _I)] + [(n, Nvfp4) for n in ("q", "k", "v", "g", "o", "gate", "up", "down")] + \
               [(n, _P) for n in ("qscale", "gscale", "sg", "su", "lr")]


SIGNATURES = [
    ("xtg_hip_open", _P, [ctypes.c_char_p] + _ERR),
    ("xtg_hip_close", None, [_P]),
    ("xtg_hip_info", _I, [_P, ctypes.c_char_p, _I]),
    ("xtg_hip_stream", _P, [_P]),
    ("xtg_hip_prepare_nvfp4", _I, [_P, ctypes.POINTER(Nvfp4)] + _ERR),
    ("xtg_hip_release_nvfp4", _I, [_P, _P] + _ERR),
    ("xtg_hip_matmul_nvfp4", _I, [_P, ctypes.POINTER(Nvfp4), _I, _P, _I, ctypes.POINTER(_P)] + _ERR),
    ("xtg_hip_matmul_nvfp4_dev", _I, [_P, ctypes.POINTER(Nvfp4), _I, _P, _I, _I, _P, _SZ] + _ERR),
    ("xtg_hip_prepare_bf16", _I, [_P, ctypes.POINTER(Bf16)] + _ERR),
    ("xtg_hip_release_bf16", _I, [_P, _P] + _ERR),
    ("xtg_hip_matmul_bf16", _I, [_P, ctypes.POINTER(Bf16), _P, _I, _P] + _ERR),
    ("xtg_hip_matmul_bf16_dev", _I, [_P, ctypes.POINTER(Bf16), _P, _I, _I, _P, _SZ] + _ERR),
    ("xtg_hip_kv_create", _P, [_P, _I, _I, _I64, _I, _I] + _ERR),
    ("xtg_hip_kv_destroy", None, [_P, _P]),
    ("xtg_hip_kv_store", _I, [_P, _P, _I64, _I, _P, _P] + _ERR),
    ("xtg_hip_kv_load", _I, [_P, _P, _I, _I64, _I64, _P, _P] + _ERR),
    ("xtg_hip_kv_bytes", _I64, [_P, _P]),
    ("xtg_hip_kv_save", _I, [_P, _P, _P, _SZ] + _ERR),
    ("xtg_hip_kv_restore", _I, [_P, _P, _P, _SZ] + _ERR),
    ("xtg_hip_kv_copy", _I, [_P, _P, _P] + _ERR),
    ("xtg_hip_nvfp4_tiles", _I, [_P, _P, _P, _SZ] + _ERR),
    ("xtg_hip_kv_release", _I, [_P, _P] + _ERR),
    ("xtg_hip_attention", _I, [_P, ctypes.POINTER(AttnArgs)] + _ERR),
    ("xtg_hip_attention_noalloc", _I, [_P, ctypes.POINTER(AttnArgs)] + _ERR),
    ("xtg_hip_qk_rope_norm", _I, [_P, _P, _P, _I, _I, _I, _I, _I64, _F, _P] + _ERR),
    ("xtg_hip_slerp_residual", _I, [_P, _P, _P, _P, _I, _I] + _ERR),
    ("xtg_hip_swiglu_norm", _I, [_P, _P, _P, _P, _P, _I, _I] + _ERR),
    ("xtg_hip_gate_norm", _I, [_P, _P, _P, _P, _I, _I] + _ERR),
    ("xtg_hip_add_norm", _I, [_P, _P, _P, _P, _I, _I] + _ERR),
    ("xtg_hip_argmax", _I, [_P, _P, _I, _I, _P] + _ERR),
    ("xtg_hip_sample", _I, [_P, _P, _I, _I, ctypes.POINTER(Sampling), _P, _P] + _ERR),
    ("xtg_hip_dory_create", _P, [_P, ctypes.POINTER(DoryConfig), ctypes.POINTER(DoryLayer), ctypes.POINTER(Nvfp4),
                                 _P] + _ERR),
    ("xtg_hip_dory_destroy", None, [_P]),
    ("xtg_hip_dory_head_bf16", _I, [_P, ctypes.POINTER(Bf16)] + _ERR),
    ("xtg_hip_dory_forward", _I, [_P, _P, _I, _I64, _P] + _ERR),
    ("xtg_hip_dory_prefill", _I, [_P, _P, _I, _I64, _I, _P] + _ERR),
    ("xtg_hip_dory_cache", _P, [_P, _I, _I]),
    ("xtg_hip_dory_snapshot", _I, [_P, _I] + _ERR),
    ("xtg_hip_dory_restore", _I, [_P, _I] + _ERR),
    ("xtg_hip_x_operand_bytes", _SZ, [_I]),
    ("xtg_hip_prep_x", _I, [_P, _P, _I, _I, _I, _P] + _ERR),
    ("xtg_hip_matmul_nvfp4_op", _I, [_P, ctypes.POINTER(Nvfp4), _I, _P, _I, _P, _SZ] + _ERR),
    ("xtg_hip_alloc", _I, [_P, _SZ, ctypes.POINTER(_P)] + _ERR),
    ("xtg_hip_release", None, [_P, _P]),
    ("xtg_hip_write", _I, [_P, _P, _SZ, _P, _SZ] + _ERR),
    ("xtg_hip_read", _I, [_P, _P, _SZ, _P, _SZ] + _ERR),
    ("xtg_hip_copy", _I, [_P, _P, _SZ, _P, _SZ, _SZ] + _ERR),
    ("xtg_hip_finish", _I, [_P] + _ERR),
    ("xtg_hip_graph_begin", _I, [_P] + _ERR),
    ("xtg_hip_graph_end", _I, [_P, ctypes.c_char_p, ctypes.POINTER(_P)] + _ERR),
    ("xtg_hip_graph_launch", _I, [_P, _P] + _ERR),
    ("xtg_hip_graph_destroy", None, [_P, _P]),
    ("xtg_hip_read_probe_partials", _SZ, [_SZ]),
    ("xtg_hip_read_probe", _I, [_P, _P, _SZ, _P] + _ERR),
    ("xtg_hip_profile", _I, [_P, _I] + _ERR),
    ("xtg_hip_profile_report", _I, [_P, ctypes.c_char_p, _I]),
]

_lib = None


class XtgError(RuntimeError):
    pass


def lib():
    """The loaded library; raises when it is not built (there is no fallback path)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise XtgError("libxtg_hip.so is not built (run __graft_entry__.build() or xtier-go_amd/build.py)")
        l = ctypes.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


def _errbuf():
    return ctypes.create_string_buffer(2048)


def _check(rc, err):
    if rc != 0:
        raise XtgError(err.value.decode(errors="replace"))


def _ptr(a):
    """Address of a numpy array or a torch tensor (device or host), or an int."""
    if a is None:
        return None
    if isinstance(a, int):
        return a
    if isinstance(a, np.ndarray):
        return a.ctypes.data
    return a.data_ptr()   # torch.Tensor


class Weight:
    """An NVFP4 weight held in host memory: codes [n][k/2] u8, scales [n][k/16] u8 (E4M3), global f32."""

    def __init__(self, codes, scales, glob=1.0):
        self.codes = np.ascontiguousarray(codes, dtype=np.uint8)
        self.scales = np.ascontiguousarray(scales, dtype=np.uint8)
        self.glob = float(glob)
        self.n_out = self.codes.shape[0]
        self.k = self.codes.shape[1] * 2
        assert self.scales.shape == (self.n_out, self.k // 16)

    def struct(self):
        return Nvfp4(self.codes.ctypes.data, self.scales.ctypes.data, self.glob, self.n_out, self.k)


def _structs(ws):
    arr = (Nvfp4 * len(ws))()
    for i, w in enumerate(ws):
        arr[i] = w.struct()
    return arr


class HipBackend:
    """One xtg_hip handle (a device, its stream and prepared weights)."""

    def __init__(self, device=0):
        err = _errbuf()
        self.h = lib().xtg_hip_open(json.dumps({"device": device}).encode(), err, len(err))
        if not self.h:
            raise XtgError(err.value.decode(errors="replace"))
        # Prepared weights are keyed by the address of their codes (as in the reference); every Weight passed in
        # is kept alive here so that no later array can reuse an address that still names a prepared copy.
        self._weights = {}

    def close(self):
        if self.h:
            lib().xtg_hip_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self):
        buf = ctypes.create_string_buffer(4096)
        n = lib().xtg_hip_info(self.h, buf, len(buf))
        if n < 0:
            raise XtgError("info failed")
        return json.loads(buf.value.decode())

    @property
    def stream(self):
        return lib().xtg_hip_stream(self.h)

    def _hold(self, ws):
        for w in ws:
            self._weights.setdefault(w.codes.ctypes.data, w)
        return _structs(ws)

    def prepare(self, w):
        err = _errbuf()
        arr = self._hold([w])
        _check(lib().xtg_hip_prepare_nvfp4(self.h, arr, err, len(err)), err)

    def nvfp4_tiles(self, w):
        """The device tile layout prepared for w (uint8, ceil(n/16) * ceil(k/128) * 1152 bytes)."""
        n, k = w.codes.shape[0], w.codes.shape[1] * 2
        out = np.empty(((n + 15) // 16) * ((k + 127) // 128) * 1152, np.uint8)
        err = _errbuf()
        _check(lib().xtg_hip_nvfp4_tiles(self.h, w.codes.ctypes.data, out.ctypes.data, out.nbytes, err, len(err)), err)
        return out

    def release_weight(self, w):
        """Drop the device copy of w (and let its host arrays go)."""
        err = _errbuf()
        key = w.codes.ctypes.data
        _check(lib().xtg_hip_release_nvfp4(self.h, key, err, len(err)), err)
        self._weights.pop(key, None)

    def matmul(self, ws, x):
        """Host-synchronous matmul_nvfp4: x float32 [m][k] -> list of float32 [m][n_i]."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        m = x.shape[0]
        ys = [np.empty((m, w.n_out), dtype=np.float32) for w in ws]
        yp = (_P * len(ws))(*[y.ctypes.data for y in ys])
        err = _errbuf()
        _check(lib().xtg_hip_matmul_nvfp4(self.h, self._hold(ws), len(ws), x.ctypes.data, m, yp, err, len(err)), err)
        return ys

    def matmul_dev(self, ws, x, x_dtype, m, y, y_offset=0):
        """Queued device matmul: x, y are device addresses (ints or torch tensors)."""
        err = _errbuf()
        _check(lib().xtg_hip_matmul_nvfp4_dev(self.h, self._hold(ws), len(ws), _ptr(x), x_dtype, m, _ptr(y), y_offset,
                                              err, len(err)), err)

    @staticmethod
    def x_operand_bytes(k):
        return lib().xtg_hip_x_operand_bytes(k)

    def prep_x(self, x, x_dtype, m, k, op):
        """Queued: the matrix-core operand of x ([m][k] on the device) into the device buffer op."""
        err = _errbuf()
        _check(lib().xtg_hip_prep_x(self.h, _ptr(x), x_dtype, m, k, _ptr(op), err, len(err)), err)

    def matmul_op(self, ws, op, m, y, y_offset=0):
        """Queued: the projections of a prepared operand into y (as matmul_dev)."""
        err = _errbuf()
        _check(lib().xtg_hip_matmul_nvfp4_op(self.h, self._hold(ws), len(ws), _ptr(op), m, _ptr(y), y_offset, err,
                                             len(err)), err)

    # ---- BF16 weights (xtg::Bf16Weight): w is a C-contiguous uint16 array [n_out][k] of BF16 bits
    def _bf16(self, w):
        assert w.dtype == np.uint16 and w.ndim == 2 and w.flags.c_contiguous
        self._weights.setdefault(w.ctypes.data, w)
        return Bf16(w.ctypes.data, w.shape[0], w.shape[1])

    def prepare_bf16(self, w):
        err = _errbuf()
        st = self._bf16(w)
        _check(lib().xtg_hip_prepare_bf16(self.h, ctypes.byref(st), err, len(err)), err)

    def release_bf16(self, w):
        err = _errbuf()
        _check(lib().xtg_hip_release_bf16(self.h, w.ctypes.data, err, len(err)), err)
        self._weights.pop(w.ctypes.data, None)

    def matmul_bf16(self, w, x):
        """Host-synchronous matmul_bf16: x float32 [m][k] -> float32 [m][n_out]."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty((x.shape[0], w.shape[0]), dtype=np.float32)
        err = _errbuf()
        st = self._bf16(w)
        _check(lib().xtg_hip_matmul_bf16(self.h, ctypes.byref(st), x.ctypes.data, x.shape[0], y.ctypes.data, err,
                                         len(err)), err)
        return y

    def matmul_bf16_dev(self, w, x, x_dtype, m, y, y_offset=0):
        """Queued device matmul_bf16: x, y are device addresses."""
        err = _errbuf()
        st = self._bf16(w)
        _check(lib().xtg_hip_matmul_bf16_dev(self.h, ctypes.byref(st), _ptr(x), x_dtype, m, _ptr(y), y_offset, err,
                                             len(err)), err)

    def alloc(self, nbytes):
        err = _errbuf()
        out = _P()
        _check(lib().xtg_hip_alloc(self.h, nbytes, ctypes.byref(out), err, len(err)), err)
        return out.value

    def release(self, mem):
        lib().xtg_hip_release(self.h, mem)

    def write(self, mem, src, offset=0):
        src = np.ascontiguousarray(src)
        err = _errbuf()
        _check(lib().xtg_hip_write(self.h, _ptr(mem), offset, src.ctypes.data, src.nbytes, err, len(err)), err)

    def read(self, mem, dst, offset=0):
        err = _errbuf()
        _check(lib().xtg_hip_read(self.h, _ptr(mem), offset, dst.ctypes.data, dst.nbytes, err, len(err)), err)
        return dst

    def copy(self, src, dst, nbytes, src_offset=0, dst_offset=0):
        err = _errbuf()
        _check(lib().xtg_hip_copy(self.h, _ptr(src), src_offset, _ptr(dst), dst_offset, nbytes, err, len(err)), err)

    def finish(self):
        err = _errbuf()
        _check(lib().xtg_hip_finish(self.h, err, len(err)), err)

    def graph_begin(self):
        err = _errbuf()
        _check(lib().xtg_hip_graph_begin(self.h, err, len(err)), err)

    def graph_end(self, name=None):
        """The captured graph (an opaque handle for graph_launch / graph_destroy)."""
        err = _errbuf()
        g = _P()
        _check(lib().xtg_hip_graph_end(self.h, name.encode() if name else None, ctypes.byref(g), err, len(err)), err)
        return g.value

    def graph_launch(self, g):
        err = _errbuf()
        _check(lib().xtg_hip_graph_launch(self.h, g, err, len(err)), err)

    def graph_destroy(self, g):
        lib().xtg_hip_graph_destroy(self.h, g)

    def profile(self, enable=True, launches=False):
        """Per-kernel event timing on (launches: also every launch's time in queue order) or off."""
        err = _errbuf()
        _check(lib().xtg_hip_profile(self.h, (2 if launches else 1) if enable else 0, err, len(err)), err)

    def profile_report(self, launches=False):
        """{kernel name: {"calls": n, "ms": total}} since the last report (waits for queued work); with launches,
        also the list [(name, ms), ...] of every launch in queue order (profiling turned on with launches=True)."""
        buf = ctypes.create_string_buffer(1 << 22)
        n = lib().xtg_hip_profile_report(self.h, buf, len(buf))
        if n < 0 or n >= len(buf):
            raise XtgError("profile report failed")
        rep = json.loads(buf.value.decode())
        if launches:
            return rep["kernels"], [tuple(x) for x in rep.get("launches", [])]
        return rep["kernels"]

    def array(self, a=None, shape=None, dtype=np.float32):
        """A device buffer owned by this backend, filled from the numpy array a (or left unset)."""
        return DeviceArray(self, a, shape, dtype)

    # ---- KV caches and attention (engine/include/xtg/kv.h)
    def kv_cache(self, kv_heads, head_dim, slots, ring=0, dtype=KV_BF16):
        return KvCache(self, kv_heads, head_dim, slots, ring, dtype)

    def attention(self, cache, q, k, v, out, n_q, pos0, heads, window=0, scale=None):
        """Queued device attention: q, k, v, out device buffers as xtg::AttnArgs."""
        sc = float(np.float32(1) / np.sqrt(np.float32(cache.head_dim))) if scale is None else float(scale)
        a = AttnArgs(n_q, pos0, heads, cache.kv_heads, cache.head_dim, window, sc, _ptr(q), _ptr(k), _ptr(v), cache.h,
                     _ptr(out))
        err = _errbuf()
        _check(lib().xtg_hip_attention(self.h, ctypes.byref(a), err, len(err)), err)

    def attention_noalloc(self, cache, q, k, v, out, n_q, pos0, heads, window=0, scale=None):
        """The same call with its partials in the device's fixed scratch (xtg_hip_attention_noalloc)."""
        sc = float(np.float32(1) / np.sqrt(np.float32(cache.head_dim))) if scale is None else float(scale)
        a = AttnArgs(n_q, pos0, heads, cache.kv_heads, cache.head_dim, window, sc, _ptr(q), _ptr(k), _ptr(v), cache.h,
                     _ptr(out))
        err = _errbuf()
        _check(lib().xtg_hip_attention_noalloc(self.h, ctypes.byref(a), err, len(err)), err)

    # ---- the Dory decode step
    def dory(self, weights):
        """A decode session over DoryWeights (xtier_go_amd.workloads); the weights stay referenced by it."""
        return DorySession(self, weights)

    # ---- row kernels (queued, device buffers)
    def qk_rope_norm(self, q, k, m, heads, kv_heads, head_dim, pos0, theta, qscale=None):
        err = _errbuf()
        _check(lib().xtg_hip_qk_rope_norm(self.h, _ptr(q), _ptr(k), m, heads, kv_heads, head_dim, pos0, theta,
                                          _ptr(qscale), err, len(err)), err)

    def slerp_residual(self, x, o, lr, rows, width):
        err = _errbuf()
        _check(lib().xtg_hip_slerp_residual(self.h, _ptr(x), _ptr(o), _ptr(lr), rows, width, err, len(err)), err)

    def swiglu_norm(self, g, u, sg, su, rows, width):
        err = _errbuf()
        _check(lib().xtg_hip_swiglu_norm(self.h, _ptr(g), _ptr(u), _ptr(sg), _ptr(su), rows, width, err, len(err)),
               err)

    def gate_norm(self, att, gate, gs, rows, width):
        err = _errbuf()
        _check(lib().xtg_hip_gate_norm(self.h, _ptr(att), _ptr(gate), _ptr(gs), rows, width, err, len(err)), err)

    def add_norm(self, a, b, out, rows, width):
        err = _errbuf()
        _check(lib().xtg_hip_add_norm(self.h, _ptr(a), _ptr(b), _ptr(out), rows, width, err, len(err)), err)

    def read_probe(self, src, nbytes, out):
        """The streaming-read probe: out (device uint32, read_probe_partials(nbytes)) gets the XOR partials of the
        nbytes at src (device)."""
        err = _errbuf()
        _check(lib().xtg_hip_read_probe(self.h, _ptr(src), nbytes, _ptr(out), err, len(err)), err)

    @staticmethod
    def read_probe_partials(nbytes):
        return int(lib().xtg_hip_read_probe_partials(nbytes))

    def argmax(self, logits, rows, n, out):
        """out[r] (device int32) = the first index of the largest of logits[r][:n] (device)."""
        err = _errbuf()
        _check(lib().xtg_hip_argmax(self.h, _ptr(logits), rows, n, _ptr(out), err, len(err)), err)

    def sample(self, logits, rows, n, u, out, temperature=1.0, top_p=1.0, top_k=0, min_p=0.0):
        """out[r] (device int32) = xtg::Sampler::sample of logits[r][:n] (device) with the uniform draw u[r] in
        [0, 1) (host; the reference's generate_canonical draw)."""
        uu = np.ascontiguousarray(u, dtype=np.float64)
        assert uu.shape == (rows,)
        p = Sampling(temperature, top_p, top_k, min_p)
        err = _errbuf()
        _check(lib().xtg_hip_sample(self.h, _ptr(logits), rows, n, ctypes.byref(p), uu.ctypes.data, _ptr(out), err,
                                    len(err)), err)


class DorySession:
    """xtg_hip_dory: forward(x, m, pos0, logits) and prefill(x, n, pos0, want, logits) on device buffers;
    cache(attn, inst) for filling contexts."""

    def __init__(self, backend, weights):
        import xtier_go_amd.workloads as wl
        self.b = backend
        self.w = weights
        cfg, layers, head = wl.dory_structs(weights, Nvfp4, DoryLayer, DoryConfig)
        self._keep = (cfg, layers, head)
        err = _errbuf()
        self.h = lib().xtg_hip_dory_create(backend.h, ctypes.byref(cfg), layers, ctypes.byref(head),
                                           weights.logit_scale.ctypes.data, err, len(err))
        if not self.h:
            raise XtgError(err.value.decode(errors="replace"))
        if getattr(weights, "head_bf16", None) is not None:   # a checkpoint's BF16 LM head
            self.set_head_bf16(weights.head_bf16)

    def destroy(self):
        if self.h:
            lib().xtg_hip_dory_destroy(self.h)
            self.h = None

    def forward(self, x, m, pos0, logits):
        """One chunk of m <= 512 rows; logits for every row."""
        err = _errbuf()
        _check(lib().xtg_hip_dory_forward(self.h, _ptr(x), m, pos0, _ptr(logits), err, len(err)), err)

    def prefill(self, x, n, pos0, want, logits=None):
        """n rows in chunks of up to 512; logits for all rows, the last or none (LOGITS_*)."""
        err = _errbuf()
        _check(lib().xtg_hip_dory_prefill(self.h, _ptr(x), n, pos0, want, _ptr(logits) if logits is not None else None,
                                          err, len(err)), err)

    def set_head_bf16(self, w):
        """A BF16 LM head (uint16 BF16 bits [vocab][hidden], kept referenced) in place of the NVFP4 one."""
        assert w.dtype == np.uint16 and w.flags.c_contiguous
        self._head_bf16 = w
        st = Bf16(w.ctypes.data, w.shape[0], w.shape[1])
        err = _errbuf()
        _check(lib().xtg_hip_dory_head_bf16(self.h, ctypes.byref(st), err, len(err)), err)

    def snapshot(self, slot):
        err = _errbuf()
        _check(lib().xtg_hip_dory_snapshot(self.h, slot, err, len(err)), err)

    def restore(self, slot):
        err = _errbuf()
        _check(lib().xtg_hip_dory_restore(self.h, slot, err, len(err)), err)

    def cache(self, attn, inst=0):
        h = lib().xtg_hip_dory_cache(self.h, attn, inst)
        if not h:
            raise XtgError("no cache %d / %d" % (attn, inst))
        c = KvCache.__new__(KvCache)
        c.b, c.h, c.owned = self.b, h, False
        c.kv_heads, c.head_dim = self.w.cfg["kv_heads"], self.w.cfg["head_dim"]
        return c


class KvCache:
    """A device KV cache (xtg_hip_kv): store from device rows, load to host, save / restore / release."""

    def __init__(self, backend, kv_heads, head_dim, slots, ring=0, dtype=KV_BF16):
        self.b = backend
        self.kv_heads, self.head_dim = kv_heads, head_dim
        self.slots = ring if ring > 0 else slots
        self.ring = ring
        self.owned = True
        err = _errbuf()
        self.h = lib().xtg_hip_kv_create(backend.h, kv_heads, head_dim, slots, ring, dtype, err, len(err))
        if not self.h:
            raise XtgError(err.value.decode(errors="replace"))

    def destroy(self):
        if self.h and self.b.h and self.owned:
            lib().xtg_hip_kv_destroy(self.b.h, self.h)
        self.h = None

    def store(self, pos, n, k, v):
        """Rows pos .. pos + n - 1 from device FP32 k, v [n][kv_heads][head_dim] (queued)."""
        err = _errbuf()
        _check(lib().xtg_hip_kv_store(self.b.h, self.h, pos, n, _ptr(k), _ptr(v), err, len(err)), err)

    def store_host(self, pos, k, v):
        """Convenience: upload FP32 host rows, then store them."""
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        dk, dv = self.b.array(k), self.b.array(v)
        self.store(pos, k.shape[0], dk, dv)
        self.b.finish()
        dk.free()
        dv.free()

    def load(self, head, p0, p1):
        k = np.empty((p1 - p0, self.head_dim), dtype=np.float32)
        v = np.empty_like(k)
        err = _errbuf()
        _check(lib().xtg_hip_kv_load(self.b.h, self.h, head, p0, p1, k.ctypes.data, v.ctypes.data, err, len(err)), err)
        return k, v

    def nbytes(self):
        return lib().xtg_hip_kv_bytes(self.b.h, self.h)

    def save(self):
        out = np.empty(self.nbytes(), dtype=np.uint8)
        err = _errbuf()
        _check(lib().xtg_hip_kv_save(self.b.h, self.h, out.ctypes.data, out.nbytes, err, len(err)), err)
        return out

    def restore(self, blob):
        blob = np.ascontiguousarray(blob, dtype=np.uint8)
        err = _errbuf()
        _check(lib().xtg_hip_kv_restore(self.b.h, self.h, blob.ctypes.data, blob.nbytes, err, len(err)), err)

    def release(self):
        err = _errbuf()
        _check(lib().xtg_hip_kv_release(self.b.h, self.h, err, len(err)), err)

    def copy_to(self, dst):
        """Device copy of this cache's whole state into dst (same shape, ring and dtype)."""
        err = _errbuf()
        _check(lib().xtg_hip_kv_copy(self.b.h, self.h, dst.h, err, len(err)), err)


class DeviceArray:
    """Device memory from xtg_hip_alloc with a numpy shape and dtype (the library's own buffers, so no other
    HIP runtime is involved)."""

    def __init__(self, backend, a=None, shape=None, dtype=np.float32):
        self.b = backend
        if a is not None:
            a = np.ascontiguousarray(a)
            shape, dtype = a.shape, a.dtype
        self.shape = tuple(shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self.ptr = backend.alloc(max(self.nbytes, 4))
        if a is not None:
            backend.write(self.ptr, a)

    def data_ptr(self):
        return self.ptr

    def upload(self, a):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes
        self.b.write(self.ptr, a)

    def numpy(self):
        out = np.empty(self.shape, dtype=self.dtype)
        return self.b.read(self.ptr, out)

    def free(self):
        if self.ptr:
            self.b.release(self.ptr)
            self.ptr = None

"""ctypes wrappers of the CPU oracle (liboracle.so) and, where it was built, of the reference engine's own CPU
kernels (_ref/libxtgref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker or the CPU baseline. The HIP library never uses it.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libxtgref.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_I64 = ctypes.c_int64


class Nvfp4(ctypes.Structure):
    _fields_ = [("codes", _P), ("scales", _P), ("glob", _F), ("n_out", _I), ("k", _I)]


class AttnArgs(ctypes.Structure):
    """xo_attn_args / xr_attn_args (the field order of xtg::AttnArgs, engine/include/xtg/kv.h:67-78)."""
    _fields_ = [("n_q", _I), ("pos0", _I64), ("heads", _I), ("kv_heads", _I), ("head_dim", _I), ("window", _I),
                ("scale", _F), ("q", _P), ("k", _P), ("v", _P), ("cache", _P), ("out", _P)]


class DoryConfig(ctypes.Structure):
    """xo_dory_config."""
    _fields_ = [(n, _I) for n in ("hidden", "ffn", "heads", "kv_heads", "head_dim", "vocab", "n_in", "n_rec", "n_out",
                                  "loops", "window", "ring_slots")] + \
               [("context", _I64), ("theta_sliding", _F), ("theta_full", _F), ("kv_dtype", _I), ("kv_mode", _I)]


class DoryLayer(ctypes.Structure):
    """xo_dory_layer."""
    _fields_ = [("kind", _I)] + [(n, Nvfp4) for n in ("q", "k", "v", "g", "o", "gate", "up", "down")] + \
               [(n, _P) for n in ("qscale", "gscale", "sg", "su", "lr")]


def _load(path, sigs):
    l = ctypes.CDLL(path)
    for name, res, args in sigs:
        f = getattr(l, name)
        f.restype = res
        f.argtypes = args
    return l


_ORACLE_SIGS = [
    ("xo_bf16_to_f32", _F, [ctypes.c_uint16]),
    ("xo_f32_to_bf16", ctypes.c_uint16, [_F]),
    ("xo_e4m3_to_f32", _F, [ctypes.c_uint8]),
    ("xo_f32_to_e4m3", ctypes.c_uint8, [_F]),
    ("xo_e4m3_bits", ctypes.c_uint8, [_F]),
    ("xo_e2m1", _F, [_I]),
    ("xo_nvfp4_row", None, [ctypes.POINTER(Nvfp4), _I, _P]),
    ("xo_matmul_nvfp4", _I, [ctypes.POINTER(Nvfp4), _I, _P, _I, ctypes.POINTER(_P), _I]),
    ("xo_matmul_bf16", _I, [_P, _I, _I, _P, _I, _P, _I]),
    ("xo_bf16_row", None, [_P, _I64, _I, _P]),
    ("xo_justnorm", None, [_P, _I, _I]),
    ("xo_slerp_residual", None, [_P, _P, _P, _I, _I]),
    ("xo_rope", None, [_P, _I, _I, _I, _I64, _F]),
    ("xo_swiglu_scaled", None, [_P, _P, _P, _P, _I, _I]),
    ("xo_rope_table", None, [_P, _I, _I, _I64, _F]),
    ("xo_qk_produce", None, [_P, _P, _I, _I, _I, _I, _I64, _F, _P]),
    ("xo_gate_norm", None, [_P, _P, _P, _I, _I]),
    ("xo_add_norm", None, [_P, _P, _P, _I, _I]),
    ("xo_argmax", _I, [_P, _I]),
    ("xo_sample", _I, [_P, _I, ctypes.c_float, ctypes.c_float, _I, ctypes.c_float, ctypes.c_double, _P]),
    ("xo_kv_create", _P, [_I, _I, _I64, _I, _I]),
    ("xo_kv_free", None, [_P]),
    ("xo_kv_slots", _I64, [_P]),
    ("xo_kv_store", _I, [_P, _I64, _I, _P, _P]),
    ("xo_kv_load", None, [_P, _I, _I64, _I64, _P, _P]),
    ("xo_kv_kdata", _P, [_P]),
    ("xo_kv_vdata", _P, [_P]),
    ("xo_kv_kscale", _P, [_P]),
    ("xo_kv_vscale", _P, [_P]),
    ("xo_attention", _I, [ctypes.POINTER(AttnArgs), _I, _I]),
    ("xo_attention_slots", _I, [ctypes.POINTER(AttnArgs), _P, _I]),
    ("xo_dory_create", _P, [ctypes.POINTER(DoryConfig), ctypes.POINTER(DoryLayer), ctypes.POINTER(Nvfp4), _P]),
    ("xo_dory_free", None, [_P]),
    ("xo_dory_cache", _P, [_P, _I, _I]),
    ("xo_dory_head_bf16", None, [_P, _P]),
    ("xo_dory_forward", _I, [_P, _P, _I, _I64, _P, _I]),
]

_REF_SIGS = [
    ("xr_e4m3_to_f32", _F, [ctypes.c_uint8]),
    ("xr_f32_to_e4m3", ctypes.c_uint8, [_F]),
    ("xr_f32_to_bf16", ctypes.c_uint16, [_F]),
    ("xr_bf16_to_f32", _F, [ctypes.c_uint16]),
    ("xr_nvfp4_row", None, [ctypes.POINTER(Nvfp4), _I, _P]),
    ("xr_matmul_nvfp4", _I, [ctypes.POINTER(Nvfp4), _I, _P, _I, ctypes.POINTER(_P), _I]),
    ("xr_matmul_bf16", _I, [_P, _I, _I, _P, _I, _P, _I]),
    ("xr_justnorm", None, [_P, _I, _I]),
    ("xr_argmax", _I, [_P, _I]),
    ("xr_sample", _I, [_P, _I, ctypes.c_float, ctypes.c_float, _I, ctypes.c_float, ctypes.c_uint64, _P]),
    ("xr_slerp_residual", None, [_P, _P, _P, _I, _I]),
    ("xr_rope", None, [_P, _I, _I, _I, _I64, _F]),
    ("xr_swiglu_scaled", None, [_P, _P, _P, _P, _I, _I]),
    ("xr_kv_create", _P, [_I, _I, _I64, _I, _I]),
    ("xr_kv_free", None, [_P]),
    ("xr_kv_store", _I, [_P, _I64, _I, _P, _P]),
    ("xr_kv_load", None, [_P, _I, _I64, _I64, _P, _P]),
    ("xr_attention", _I, [ctypes.POINTER(AttnArgs), _I]),
    ("xr_dory_open", _P, [ctypes.c_char_p, ctypes.c_char_p, _I, ctypes.POINTER(_I), ctypes.c_char_p, _I]),
    ("xr_dory_close", None, [_P]),
    ("xr_dory_forward", _I, [_P, _P, _I, _I, _P, ctypes.c_char_p, _I]),
    ("xr_dory_n_past", _I64, [_P]),
    ("xr_dory_rewind", _I, [_P, _I64]),
    ("xr_dory_snapshot", None, [_P, _I]),
    ("xr_dory_restore", _I, [_P, _I]),
]

_oracle = None
_ref = None


def oracle():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError("oracle/liboracle.so is not built (make -C oracle)")
        _oracle = _load(ORACLE_SO, _ORACLE_SIGS)
    return _oracle


def ref_available():
    return os.path.exists(REF_SO)


def ref():
    global _ref
    if _ref is None:
        _ref = _load(REF_SO, _REF_SIGS)
    return _ref


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _wstructs(ws):
    arr = (Nvfp4 * len(ws))()
    for i, (codes, scales, glob) in enumerate(ws):
        arr[i] = Nvfp4(codes.ctypes.data, scales.ctypes.data, float(glob), codes.shape[0], codes.shape[1] * 2)
    return arr


def matmul_nvfp4(ws, x, threads=8, use_ref=False):
    """ws: list of (codes, scales, global); x float32 [m][k]. Returns a list of float32 [m][n_i]."""
    x = _f32(x)
    m = x.shape[0]
    for codes, scales, _ in ws:
        assert codes.flags.c_contiguous and scales.flags.c_contiguous
    ys = [np.empty((m, c.shape[0]), dtype=np.float32) for c, _, _ in ws]
    yp = (_P * len(ws))(*[y.ctypes.data for y in ys])
    st = _wstructs(ws)
    if use_ref:
        rc = ref().xr_matmul_nvfp4(st, len(ws), x.ctypes.data, m, yp, threads)
    else:
        rc = oracle().xo_matmul_nvfp4(st, len(ws), x.ctypes.data, m, yp, threads)
    if rc != 0:
        raise ValueError("matmul_nvfp4 rejected its arguments")
    return ys


def matmul_bf16(w, x, threads=8, use_ref=False):
    """w: uint16 BF16 bits [n_out][k]; x float32 [m][k]. Returns float32 [m][n_out]."""
    w = np.ascontiguousarray(w, dtype=np.uint16)
    x = _f32(x)
    m, (n, k) = x.shape[0], w.shape
    assert x.shape[1] == k
    y = np.empty((m, n), dtype=np.float32)
    f = ref().xr_matmul_bf16 if use_ref else oracle().xo_matmul_bf16
    if f(w.ctypes.data, n, k, x.ctypes.data, m, y.ctypes.data, threads) != 0:
        raise ValueError("matmul_bf16 rejected its arguments")
    return y


def nvfp4_row(codes, scales, glob, n, use_ref=False):
    st = _wstructs([(codes, scales, glob)])
    out = np.empty(codes.shape[1] * 2, dtype=np.float32)
    (ref().xr_nvfp4_row if use_ref else oracle().xo_nvfp4_row)(st, n, out.ctypes.data)
    return out


def justnorm(x, use_ref=False):
    x = _f32(x).copy()
    rows = x.shape[0] if x.ndim > 1 else 1
    (ref().xr_justnorm if use_ref else oracle().xo_justnorm)(x.ctypes.data, rows, x.shape[-1])
    return x


def slerp_residual(a, b, lr, use_ref=False):
    a = _f32(a).copy()
    b = _f32(b)
    lr = _f32(lr)
    rows = a.shape[0] if a.ndim > 1 else 1
    (ref().xr_slerp_residual if use_ref else oracle().xo_slerp_residual)(a.ctypes.data, b.ctypes.data, lr.ctypes.data,
                                                                         rows, a.shape[-1])
    return a


def rope(x, heads, head_dim, pos0, theta, use_ref=False):
    """x float32 [rows][heads][head_dim] (copied)."""
    x = _f32(x).copy()
    rows = x.size // (heads * head_dim)
    (ref().xr_rope if use_ref else oracle().xo_rope)(x.ctypes.data, rows, heads, head_dim, pos0, theta)
    return x


def rope_table(m, head_dim, pos0, theta):
    cs = np.empty((2 * m, head_dim // 2), dtype=np.float32)
    oracle().xo_rope_table(cs.ctypes.data, m, head_dim, pos0, theta)
    return cs


def swiglu_scaled(g, u, sg, su, use_ref=False):
    g = _f32(g).copy()
    u = _f32(u)
    rows = g.shape[0] if g.ndim > 1 else 1
    (ref().xr_swiglu_scaled if use_ref else oracle().xo_swiglu_scaled)(g.ctypes.data, u.ctypes.data, _f32(sg).ctypes.data,
                                                                       _f32(su).ctypes.data, rows, g.shape[-1])
    return g


def gate_norm(att, gate, gs):
    att = _f32(att).copy()
    rows = att.shape[0] if att.ndim > 1 else 1
    oracle().xo_gate_norm(att.ctypes.data, _f32(gate).ctypes.data, _f32(gs).ctypes.data, rows, att.shape[-1])
    return att


def argmax(x, use_ref=False):
    """xtg::argmax (sampler.cpp:8-13) of each row of x float32 [rows][n] -> int32 [rows]."""
    x = np.atleast_2d(_f32(x))
    fn = ref().xr_argmax if use_ref else oracle().xo_argmax
    return np.array([fn(x[r].ctypes.data, x.shape[1]) for r in range(x.shape[0])], np.int32)


def sample(x, u, temperature=1.0, top_p=1.0, top_k=0, min_p=0.0):
    """xtg::Sampler::sample (sampler.cpp:40-94) of each row of x float32 [rows][n] with draws u [rows] ->
    (tokens int32 [rows], margins float64 [rows]: how close, relative to the total, r or the top_p target came to
    a running-sum boundary)."""
    x = np.atleast_2d(_f32(x))
    toks, margins = np.empty(x.shape[0], np.int32), np.empty(x.shape[0])
    m = ctypes.c_double()
    for r in range(x.shape[0]):
        toks[r] = oracle().xo_sample(x[r].ctypes.data, x.shape[1], temperature, top_p, top_k, min_p, float(u[r]),
                                     ctypes.byref(m))
        margins[r] = m.value
    return toks, margins


def sample_ref(x, seed, temperature=1.0, top_p=1.0, top_k=0, min_p=0.0):
    """The reference Sampler(seed) on one row x float32 [n] -> (token, the draw u it used)."""
    x = _f32(x)
    u = ctypes.c_double()
    t = ref().xr_sample(x.ctypes.data, x.shape[-1], temperature, top_p, top_k, min_p, seed, ctypes.byref(u))
    return t, u.value


def add_norm(a, b=None):
    a = _f32(a)
    out = np.empty_like(a)
    rows = a.shape[0] if a.ndim > 1 else 1
    oracle().xo_add_norm(a.ctypes.data, _f32(b).ctypes.data if b is not None else None, out.ctypes.data, rows,
                         a.shape[-1])
    return out


def qk_produce(q, k, heads, kv_heads, head_dim, pos0, theta, qscale):
    q = _f32(q).copy()
    k = _f32(k).copy()
    m = q.size // (heads * head_dim)
    oracle().xo_qk_produce(q.ctypes.data, k.ctypes.data, m, heads, kv_heads, head_dim, pos0, theta,
                           _f32(qscale).ctypes.data)
    return q, k


class KvCache:
    """The oracle's (or the reference's) KvCache: kv.h:21-62."""

    def __init__(self, kv_heads, head_dim, slots, ring=0, fp8=False, use_ref=False):
        self.use_ref = use_ref
        self.kv_heads, self.head_dim = kv_heads, head_dim
        self.slots = ring if ring > 0 else slots
        self.ring = ring
        if use_ref:
            self.h = ref().xr_kv_create(kv_heads, head_dim, slots, ring, 1 if fp8 else 0)
        else:
            self.h = oracle().xo_kv_create(kv_heads, head_dim, slots, ring, 1 if fp8 else 0)
        if not self.h:
            raise ValueError("KV cache creation failed")

    def __del__(self):
        try:
            if self.h and not getattr(self, "_borrowed", False):
                (ref().xr_kv_free if self.use_ref else oracle().xo_kv_free)(self.h)
            self.h = None
        except Exception:
            pass

    def store(self, pos, k, v):
        k = _f32(k)
        v = _f32(v)
        n = k.shape[0]
        f = ref().xr_kv_store if self.use_ref else oracle().xo_kv_store
        if f(self.h, pos, n, k.ctypes.data, v.ctypes.data) != 0:
            raise ValueError("KV cache full")

    def load(self, h, p0, p1):
        k = np.empty((p1 - p0, self.head_dim), dtype=np.float32)
        v = np.empty_like(k)
        (ref().xr_kv_load if self.use_ref else oracle().xo_kv_load)(self.h, h, p0, p1, k.ctypes.data, v.ctypes.data)
        return k, v

    def scales(self):
        """An FP8 cache's K and V scales [slots][kv_heads] (copies)."""
        n = self.slots * self.kv_heads
        out = []
        for f in (oracle().xo_kv_kscale, oracle().xo_kv_vscale):
            p = f(self.h)
            if not p:
                raise ValueError("not an FP8 cache")
            out.append(np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), (n,)).copy()
                       .reshape(self.slots, self.kv_heads))
        return out[0], out[1]


def attention(q, k, v, cache, pos0, heads, kv_heads, head_dim, window=0, scale=None, pool_size=8, threads=8,
              slot_pos=None):
    """q [n_q][heads][d], k / v [n_q][kv_heads][d] float32; returns out [n_q][heads][d]. With slot_pos (int64 per
    ring slot) the ring mask is taken from the stored positions (xo_attention_slots)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    n_q = q.shape[0]
    out = np.empty((n_q, heads, head_dim), dtype=np.float32)
    sc = float(scale) if scale is not None else float(np.float32(1) / np.sqrt(np.float32(head_dim)))
    a = AttnArgs(n_q, pos0, heads, kv_heads, head_dim, window, sc, q.ctypes.data, k.ctypes.data, v.ctypes.data,
                 cache.h, out.ctypes.data)
    if cache.use_ref:
        rc = ref().xr_attention(ctypes.byref(a), pool_size)
    elif slot_pos is not None:
        sp = np.ascontiguousarray(slot_pos, dtype=np.int64)
        rc = oracle().xo_attention_slots(ctypes.byref(a), sp.ctypes.data, threads)
    else:
        rc = oracle().xo_attention(ctypes.byref(a), pool_size, threads)
    if rc != 0:
        raise ValueError("attention rejected its arguments")
    return out


class Dory:
    """The oracle's decode step (packs/dory/dory.cpp:467-578) over DoryWeights (xtier-go_amd/workloads.py)."""

    def __init__(self, weights, wl):
        self.w = weights
        cfg, layers, head = wl.dory_structs(weights, Nvfp4, DoryLayer, DoryConfig)
        self._keep = (cfg, layers, head)
        self.h = oracle().xo_dory_create(ctypes.byref(cfg), layers, ctypes.byref(head), weights.logit_scale.ctypes.data)
        if getattr(weights, "head_bf16", None) is not None:   # a checkpoint's BF16 LM head
            self.set_head_bf16(weights.head_bf16)

    def __del__(self):
        try:
            if self.h:
                oracle().xo_dory_free(self.h)
                self.h = None
        except Exception:
            pass

    def forward(self, x, pos0, threads=8):
        """x float32 [m][hidden] -> logits float32 [m][vocab]."""
        x = _f32(x)
        m = x.shape[0]
        out = np.empty((m, self.w.cfg["vocab"]), dtype=np.float32)
        oracle().xo_dory_forward(self.h, x.ctypes.data, m, pos0, out.ctypes.data, threads)
        return out

    def set_head_bf16(self, w):
        """A BF16 LM head (uint16 BF16 bits [vocab][hidden], kept referenced) in place of the NVFP4 one."""
        self._head_bf16 = np.ascontiguousarray(w, dtype=np.uint16)
        oracle().xo_dory_head_bf16(self.h, self._head_bf16.ctypes.data)

    def cache(self, attn, inst=0):
        """The KvCache of attention sublayer `attn`, loop `inst` (owned by the model)."""
        c = KvCache.__new__(KvCache)
        c.use_ref = False
        c.kv_heads, c.head_dim = self.w.cfg["kv_heads"], self.w.cfg["head_dim"]
        c.h = oracle().xo_dory_cache(self.h, attn, inst)
        c.slots, c.ring = None, None
        c._borrowed = True
        return c


class RefDory:
    """The reference's own Dory pack (packs/dory/dory.cpp), compiled into oracle/_ref: load_model on a checkpoint
    directory (config.json + model.safetensors) with launch options, then one session driven as the server drives it
    (engine/include/xtg/model.h:31-63). Tokens in, logits out; positions advance with every forward."""

    LOGITS = {"none": 0, "last": 1, "all": 2}

    def __init__(self, path, options=None, threads=8):
        import json
        err = ctypes.create_string_buffer(512)
        vocab = _I(0)
        self.h = ref().xr_dory_open(path.encode(), json.dumps(options or {}).encode(), threads, ctypes.byref(vocab),
                                    err, len(err))
        if not self.h:
            raise RuntimeError("reference Dory: " + err.value.decode())
        self.vocab = vocab.value

    def close(self):
        if self.h:
            ref().xr_dory_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward(self, tokens, want="all"):
        """Session::forward over `tokens`: logits [rows][vocab] of every row ("all"), the last ("last") or none."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        rows = {"none": 0, "last": 1, "all": len(t)}[want]
        out = np.empty((max(rows, 1), self.vocab), dtype=np.float32)
        err = ctypes.create_string_buffer(512)
        got = ref().xr_dory_forward(self.h, t.ctypes.data, len(t), self.LOGITS[want], out.ctypes.data, err, len(err))
        if got < 0:
            raise RuntimeError("reference Dory forward: " + err.value.decode())
        assert got == rows, (got, rows)
        return out[:rows]

    @property
    def n_past(self):
        return int(ref().xr_dory_n_past(self.h))

    def rewind(self, n):
        return bool(ref().xr_dory_rewind(self.h, n))

    def snapshot(self, slot):
        ref().xr_dory_snapshot(self.h, slot)

    def restore(self, slot):
        return bool(ref().xr_dory_restore(self.h, slot))

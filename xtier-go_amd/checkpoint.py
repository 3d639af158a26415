"""A Dory checkpoint in ModelOpt's NVFP4 layout, read where it lies on disk.

The reference's DoryModel constructor (packs/dory/dory.cpp:316-364, 417-428) maps model.safetensors
(engine/src/safetensors.cpp:36-71) and hands the backend pointers into the map: each projection is three tensors,
`<name>.weight` U8 [n][k/2] (E2M1 codes, low nibble first), `<name>.weight_scale` F8_E4M3 [n][k/16] and
`<name>.weight_scale_2` F32 [] -- exactly xtg_nvfp4's fields -- so prepare() takes them as they are and repacks
on the device. The per-layer BF16 vectors are widened and folded as the constructor folds them, config.json is
checked as parse_config (dory.cpp:77-134) checks it, and the BF16 LM head and embedding table stay views into
the map.

DoryCheckpoint offers the interface the package's DorySession takes (cfg, kinds, layers, head, logit_scale) plus
head_bf16 and embed(tokens).
"""
import json
import math
import mmap
import os
import struct

import numpy as np

# safetensors dtype tags -> element type of the numpy view (BF16 and the FP8 formats as their raw bits)
DTYPES = {"F64": np.float64, "F32": np.float32, "F16": np.float16, "BF16": np.uint16, "I64": np.int64,
          "U64": np.uint64, "I32": np.int32, "U32": np.uint32, "I16": np.int16, "U16": np.uint16, "I8": np.int8,
          "U8": np.uint8, "BOOL": np.bool_, "F8_E4M3": np.uint8, "F8_E5M2": np.uint8}

MLP, SLIDING, FULL = 0, 1, 2
KV_BF16, KV_FP8 = 0, 1
KV_MODES = {"per_loop": 0, "last_loop": 1}   # xtg_dory_config.kv_mode
REWIND_SLACK = 16   # ring slots beyond the window (dory.cpp:43, 449)


class CheckpointError(ValueError):
    pass


def _check(cond, msg):
    if not cond:
        raise CheckpointError(msg)


class SafeTensors:
    """A safetensors file mapped read-only (engine/src/safetensors.cpp:36-71): an 8-byte little-endian header
    length, a JSON header {name: {dtype, shape, data_offsets}}, then the data. Tensors are numpy views into the
    map (no copy); the map lives as long as this object or any view."""

    def __init__(self, path):
        self.path = path
        with open(path, "rb") as f:
            size = os.fstat(f.fileno()).st_size
            _check(size >= 8, "%s: too small for a safetensors file" % path)
            self._map = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        (hlen,) = struct.unpack("<Q", self._map[:8])
        _check(0 < hlen and 8 + hlen <= size, "%s: bad header length %d" % (path, hlen))
        header = json.loads(bytes(self._map[8:8 + hlen]))
        base, data_len = 8 + hlen, size - 8 - hlen
        self.tensors = {}
        for name, t in header.items():
            if name == "__metadata__":
                continue
            dtype, shape, off = t["dtype"], tuple(int(d) for d in t["shape"]), t["data_offsets"]
            _check(len(off) == 2 and 0 <= off[0] <= off[1] <= data_len, "%s: bad offsets for %s" % (path, name))
            nbytes = int(off[1]) - int(off[0])
            eb = np.dtype(DTYPES[dtype]).itemsize if dtype in DTYPES else 0
            _check(eb == 0 or math.prod(shape) * eb == nbytes,
                   "%s: %s has %d bytes for shape %s" % (path, name, nbytes, shape))
            self.tensors[name] = (dtype, shape, base + int(off[0]), nbytes)

    def has(self, name):
        return name in self.tensors

    def get(self, name, dtype=None, shape=None):
        """The tensor as a read-only numpy view; raises naming it when it is missing or not of this dtype / shape
        (SafeTensors::get, safetensors.cpp:98-111)."""
        _check(name in self.tensors, "%s: no tensor %s" % (self.path, name))
        dt, sh, start, nbytes = self.tensors[name]
        _check(dtype is None or dt == dtype, "%s: %s is %s, expected %s" % (self.path, name, dt, dtype))
        _check(shape is None or sh == tuple(shape), "%s: %s has shape %s" % (self.path, name, sh))
        _check(dt in DTYPES, "%s: %s has the unsupported dtype %s" % (self.path, name, dt))
        return np.frombuffer(self._map, dtype=DTYPES[dt], count=math.prod(sh), offset=start).reshape(sh)


def bf16_to_f32(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def parse_config(c, where):
    """config.json of a Dory checkpoint, checked as parse_config does (dory.cpp:77-134)."""
    def need(key):
        _check(key in c and c[key] is not None, "%s: config.json has no %s" % (where, key))
        return c[key]

    _check(c.get("model_type", "") == "dory", "%s: not a Dory checkpoint" % where)
    k = dict(hidden=int(need("hidden_size")), ffn=int(need("intermediate_size")),
             heads=int(need("num_attention_heads")), kv_heads=int(need("num_key_value_heads")),
             head_dim=int(need("head_dim")), vocab=int(need("vocab_size")), layers=int(need("num_hidden_layers")),
             n_in=int(need("n_input_layers")), n_rec=int(need("n_recurrent_layers")),
             n_out=int(need("n_output_layers")), window=int(c.get("sliding_window") or 0),
             default_loops=int(c.get("n_recurrent_loops") or 1),
             default_kv_mode=c.get("recurrent_kv_cache_mode") or "per_loop",
             max_pos=int(need("max_position_embeddings")), init_range=np.float32(need("initializer_range")),
             alpha_init=np.float32(need("ngpt_alpha_init")))
    g0 = c.get("attention_output_gate_logit_scale_init")
    k["gate_init"] = np.float32(math.sqrt(k["hidden"])) if g0 is None else np.float32(g0)
    _check(k["n_in"] + k["n_rec"] + k["n_out"] == k["layers"],
           "%s: input + recurrent + output layers != %d" % (where, k["layers"]))
    _check(k["heads"] % k["kv_heads"] == 0 and k["head_dim"] % 2 == 0, "%s: unsupported attention shape" % where)
    _check(not c.get("attention_bias", False) and not c.get("mlp_bias", False), "%s: Dory has no biases" % where)
    _check(c.get("hidden_act", "silu") == "silu" and not c.get("tie_word_embeddings", False),
           "%s: Dory uses SiLU and untied embeddings" % where)
    names = {"mlp": MLP, "sliding_attention": SLIDING, "full_attention": FULL}
    kinds = []
    for t in need("layer_types"):
        _check(t in names, "%s: unknown layer type %s" % (where, t))
        kinds.append(names[t])
    _check(len(kinds) == k["layers"], "%s: layer_types has %d entries" % (where, len(kinds)))
    rope = need("rope_parameters")
    theta = {SLIDING: 0.0, FULL: 0.0}
    for kind, key in ((SLIDING, "sliding_attention"), (FULL, "full_attention")):
        if key not in rope:
            continue
        r = rope[key]
        _check(r.get("rope_type", "default") == "default" and r.get("partial_rotary_factor", 1.0) == 1.0,
               "%s: only default full-width RoPE is supported" % where)
        theta[kind] = float(np.float32(r["rope_theta"]))
    for t in kinds:
        _check(t == MLP or theta[t] > 0, "%s: a layer type has no rope_theta" % where)
    _check(k["window"] > 0 or SLIDING not in kinds, "%s: sliding layers without a window" % where)
    q = c.get("quantization_config") or {}
    _check(q.get("quant_algo", "") == "W4A16_NVFP4",
           "%s: only the W4A16_NVFP4 (ModelOpt) checkpoint is supported" % where)
    return k, kinds, theta


class DoryCheckpoint:
    """A Dory checkpoint directory (config.json + model.safetensors) in ModelOpt's W4A16_NVFP4 layout, read as the
    reference's DoryModel constructor reads it (dory.cpp:316-364, 417-428). NVFP4 projections are views into the
    mapped file; the vectors are folded as the constructor folds them:
      logit_scale / init_range; qscale = (sqk * sqrt(head_dim) / init_range)^2; gscale = (s_gate * sqrt(gate_init) /
      init_range)^2; sg, su * sqrt(hidden); lr = |alpha * alpha_init / init_range|.
    Options as the pack's (dory.cpp:136-170): loops (default n_recurrent_loops), kv_mode ("per_loop" or
    "last_loop"; default the checkpoint's recurrent_kv_cache_mode), kv_dtype (FP8 by default), context (32768),
    ring_slots (window + 16 by default; the NPU layout uses window + 64)."""

    def __init__(self, path, context=32768, kv_dtype=KV_FP8, loops=None, ring_slots=None, kv_mode=None):
        d = path if os.path.isdir(path) else os.path.dirname(path)
        with open(os.path.join(d, "config.json")) as f:
            k, kinds, theta = parse_config(json.load(f), d)
        loops = k["default_loops"] if loops is None else int(loops)
        _check(1 <= loops <= 4, "loops: %d (1..4)" % loops)
        kv_mode = k["default_kv_mode"] if kv_mode is None else kv_mode
        _check(kv_mode in KV_MODES, "kv_mode: %s (per_loop | last_loop)" % kv_mode)
        _check(256 <= context <= k["max_pos"], "context: %d (256..%d)" % (context, k["max_pos"]))
        self.st = SafeTensors(os.path.join(d, "model.safetensors"))
        H, F, V = k["hidden"], k["ffn"], k["vocab"]
        Q, KV = k["heads"] * k["head_dim"], k["kv_heads"] * k["head_dim"]
        self.kinds = kinds
        self.cfg = dict(hidden=H, ffn=F, heads=k["heads"], kv_heads=k["kv_heads"], head_dim=k["head_dim"],
                        vocab=V, n_in=k["n_in"], n_rec=k["n_rec"], n_out=k["n_out"], loops=loops,
                        window=k["window"], ring_slots=int(ring_slots or k["window"] + REWIND_SLACK),
                        theta_sliding=theta[SLIDING], theta_full=theta[FULL], context=int(context),
                        kv_dtype=int(kv_dtype), kv_mode=KV_MODES[kv_mode])
        f32 = np.float32
        self.embed_table = self.st.get("backbone.embeddings.weight", "BF16", (V, H))
        self.head_bf16 = self.st.get("lm_head.weight", "BF16", (V, H))
        self.head = None   # the checkpoint's head is BF16 (set on the session by head_bf16)
        self.logit_scale = (self.vec("lm_head.logit_scale", V) / k["init_range"]).astype(f32)
        alpha_scale = f32(k["alpha_init"] / k["init_range"])
        sqk_factor = f32(f32(math.sqrt(float(k["head_dim"]))) / k["init_range"])
        gate_factor = f32(f32(math.sqrt(float(k["gate_init"]))) / k["init_range"])
        suv_factor = f32(math.sqrt(float(H)))
        self.layers = []
        for i, kind in enumerate(kinds):
            p = "backbone.layers.%d." % i
            L = {"kind": kind}
            if kind == MLP:
                L["gate"] = self.nvfp4(p + "mixer.gate_proj", F, H)
                L["up"] = self.nvfp4(p + "mixer.up_proj", F, H)
                L["down"] = self.nvfp4(p + "mixer.down_proj", H, F)
                L["sg"] = (self.vec(p + "mixer.suv_gate", F) * suv_factor).astype(f32)
                L["su"] = (self.vec(p + "mixer.suv_up", F) * suv_factor).astype(f32)
                lr = self.vec(p + "mlp_alpha", H)
            else:
                L["q"] = self.nvfp4(p + "mixer.q_proj", Q, H)
                L["k"] = self.nvfp4(p + "mixer.k_proj", KV, H)
                L["v"] = self.nvfp4(p + "mixer.v_proj", KV, H)
                L["g"] = self.nvfp4(p + "mixer.g_proj", Q, H)
                L["o"] = self.nvfp4(p + "mixer.o_proj", H, Q)
                s = self.vec(p + "mixer.sqk", Q) * sqk_factor
                L["qscale"] = (s * s).astype(f32)
                s = self.vec(p + "mixer.s_gate", Q) * gate_factor
                L["gscale"] = (s * s).astype(f32)
                lr = self.vec(p + "attn_alpha", H)
            L["lr"] = np.abs(lr * alpha_scale).astype(f32)
            self.layers.append(L)

    def nvfp4(self, name, n_out, k):
        """(codes, scales, global) views of a ModelOpt NVFP4 projection (DoryModel::nvfp4, dory.cpp:417-428)."""
        codes = self.st.get(name + ".weight", "U8", (n_out, k // 2))
        scales = self.st.get(name + ".weight_scale", "F8_E4M3", (n_out, k // 16))
        glob = float(self.st.get(name + ".weight_scale_2", "F32", ())[()])
        return codes, scales, glob

    def vec(self, name, n):
        """A BF16 vector widened to FP32 (DoryModel::bf16_vec, dory.cpp:429-438)."""
        return bf16_to_f32(self.st.get(name, "BF16", (n,)))

    def embed(self, tokens):
        """The embedding rows of `tokens` as FP32 [n][hidden] (run_chunk's bf16_row, dory.cpp:523-526)."""
        t = np.asarray(tokens, np.int64)
        _check(((t >= 0) & (t < self.cfg["vocab"])).all(), "token out of range")
        return bf16_to_f32(self.embed_table[t])

    def n_attn(self):
        return sum(1 for k in self.kinds if k != MLP)

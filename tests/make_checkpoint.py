"""Writes a small synthetic Dory checkpoint in ModelOpt's W4A16_NVFP4 layout (config.json + model.safetensors), with
the tensor names, dtypes and shapes the reference's DoryModel constructor reads (packs/dory/dory.cpp:77-134,
316-364, 417-428). The file is written by the safetensors library from torch tensors, so the BF16 and F8_E4M3
dtype tags are the library's own. Run as a separate process (python tests/make_checkpoint.py OUT_DIR SEED [VARIANT])
so that torch's HIP runtime never shares a process with the kernel library. VARIANT "tiny" (the default: 4 q / 2 KV
heads of 64) or "d256" (4 q heads over one KV head of 256, the real Dory 4B's head size and group of 4 q heads per
KV head, docs/dory.md:13, with the shipped card's last_loop KV mode, configs/dory4b-nvfp4-sm8750/card.json).

Raw values are drawn so that the folded vectors land where the synthetic models' do: qscale, gscale ~ U(0.5, 1.5),
sg, su ~ U(5, 15), lr ~ U(0.02, 0.1), logit_scale ~ U(0.5, 1.5).
"""
import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "xtier-go_amd"))
import workloads as wl  # noqa: E402

CONFIG = {
    "model_type": "dory", "hidden_size": 256, "intermediate_size": 512, "num_attention_heads": 4,
    "num_key_value_heads": 2, "head_dim": 64, "vocab_size": 1000, "num_hidden_layers": 8, "n_input_layers": 2,
    "n_recurrent_layers": 4, "n_output_layers": 2, "sliding_window": 48, "n_recurrent_loops": 2,
    "recurrent_kv_cache_mode": "per_loop", "max_position_embeddings": 4096, "initializer_range": 0.02,
    "ngpt_alpha_init": 0.05, "hidden_act": "silu", "tie_word_embeddings": False, "attention_bias": False,
    "mlp_bias": False,
    "rope_parameters": {"sliding_attention": {"rope_type": "default", "rope_theta": 10000.0},
                        "full_attention": {"rope_type": "default", "rope_theta": 1000000.0}},
    "quantization_config": {"quant_algo": "W4A16_NVFP4"},
}
VARIANTS = {
    "tiny": {},
    "d256": {"hidden_size": 512, "intermediate_size": 1024, "num_attention_heads": 4, "num_key_value_heads": 1,
             "head_dim": 256, "recurrent_kv_cache_mode": "last_loop"},
}


def layer_types(n):
    out, a = [], 0
    for l in range(n):
        if l % 2 == 0:
            out.append("full_attention" if a % 4 == 3 else "sliding_attention")
            a += 1
        else:
            out.append("mlp")
    return out


def main(out_dir, seed, variant="tiny"):
    import torch
    from safetensors.torch import save_file

    c = dict(CONFIG, **VARIANTS[variant])
    c["layer_types"] = layer_types(c["num_hidden_layers"])
    H, F, V = c["hidden_size"], c["intermediate_size"], c["vocab_size"]
    Q, KV = c["num_attention_heads"] * c["head_dim"], c["num_key_value_heads"] * c["head_dim"]
    ir, ai = c["initializer_range"], c["ngpt_alpha_init"]
    rng = np.random.default_rng(seed)

    def bf16(x):
        return torch.from_numpy(wl.f32_to_bf16(np.asarray(x, np.float32)).view(np.int16)).view(torch.bfloat16)

    t = {}
    target = {}   # the folded values each raw vector was drawn for

    def proj(name, n, k):
        codes, scales, glob = wl.nvfp4_weight(rng, n, k)
        t[name + ".weight"] = torch.from_numpy(codes)
        t[name + ".weight_scale"] = torch.from_numpy(scales).view(torch.float8_e4m3fn)
        t[name + ".weight_scale_2"] = torch.tensor(np.float32(glob * rng.uniform(0.5, 2.0)))

    t["backbone.embeddings.weight"] = bf16(rng.standard_normal((V, H)) / math.sqrt(H))
    t["lm_head.weight"] = bf16(rng.standard_normal((V, H)))
    target["logit_scale"] = rng.uniform(0.5, 1.5, V)
    t["lm_head.logit_scale"] = bf16(target["logit_scale"] * ir)
    sqk_f = math.sqrt(c["head_dim"]) / ir
    gate_f = math.sqrt(math.sqrt(H)) / ir
    for i, kind in enumerate(c["layer_types"]):
        p = "backbone.layers.%d." % i
        if kind == "mlp":
            proj(p + "mixer.gate_proj", F, H)
            proj(p + "mixer.up_proj", F, H)
            proj(p + "mixer.down_proj", H, F)
            for key, name, n, lo, hi in (("sg", "mixer.suv_gate", F, 5, 15), ("su", "mixer.suv_up", F, 5, 15)):
                target["%d.%s" % (i, key)] = rng.uniform(lo, hi, n)
                t[p + name] = bf16(target["%d.%s" % (i, key)] / math.sqrt(H))
            target["%d.lr" % i] = rng.uniform(0.02, 0.1, H)
            t[p + "mlp_alpha"] = bf16(target["%d.lr" % i] * ir / ai * rng.choice([-1, 1], H))
        else:
            for name, n in (("q", Q), ("k", KV), ("v", KV), ("g", Q)):
                proj(p + "mixer.%s_proj" % name, n, H)
            proj(p + "mixer.o_proj", H, Q)
            for key, name, f in (("qscale", "mixer.sqk", sqk_f), ("gscale", "mixer.s_gate", gate_f)):
                target["%d.%s" % (i, key)] = rng.uniform(0.5, 1.5, Q)
                t[p + name] = bf16(np.sqrt(target["%d.%s" % (i, key)]) / f)
            target["%d.lr" % i] = rng.uniform(0.02, 0.1, H)
            t[p + "attn_alpha"] = bf16(target["%d.lr" % i] * ir / ai)
    os.makedirs(out_dir, exist_ok=True)
    save_file(t, os.path.join(out_dir, "model.safetensors"), metadata={"format": "pt"})
    with open(os.path.join(out_dir, "config.json"), "w") as f:
        json.dump(c, f, indent=1)
    np.savez(os.path.join(out_dir, "folded_targets.npz"), **target)
    # the raw bytes of every tensor, for checking a reader against the library's writer
    np.savez(os.path.join(out_dir, "raw_bytes.npz"),
             **{k: v.contiguous().view(torch.uint8).reshape(-1).numpy() if v.dim() else
                np.frombuffer(v.numpy().tobytes(), np.uint8) for k, v in t.items()})


if __name__ == "__main__":
    main(sys.argv[1], int(sys.argv[2]) if len(sys.argv) > 2 else 0, sys.argv[3] if len(sys.argv) > 3 else "tiny")

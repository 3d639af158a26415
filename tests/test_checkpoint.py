"""Ingestion of a Dory checkpoint in ModelOpt's NVFP4 layout (xtier-go_amd/checkpoint.py): the safetensors reader
against the bytes the safetensors library wrote (BF16, F8_E4M3, U8, F32 scalars), its refusals
(engine/src/safetensors.cpp:36-111), config.json's checks (packs/dory/dory.cpp:77-134) and the folding of the
vectors (dory.cpp:328-364), pinned by the values the raw vectors were drawn for (a dropped factor, a missing square
or a missing absolute value misses them by far more than BF16 rounding)."""
import json
import os

import numpy as np
import pytest


def test_reader_matches_written_bytes(ck, ckpt_dir):
    st = ck.SafeTensors(os.path.join(ckpt_dir, "model.safetensors"))
    raw = np.load(os.path.join(ckpt_dir, "raw_bytes.npz"))
    assert set(st.tensors) == set(raw.files)
    for name in raw.files:
        assert np.array_equal(np.frombuffer(st.get(name).tobytes(), np.uint8), raw[name]), name
    assert {st.tensors[n][0] for n in st.tensors} == {"BF16", "F8_E4M3", "U8", "F32"}
    assert st.get("backbone.layers.0.mixer.q_proj.weight_scale_2", "F32", ()).shape == ()


def test_reader_refusals(ck, ckpt_dir, tmp_path):
    st = ck.SafeTensors(os.path.join(ckpt_dir, "model.safetensors"))
    with pytest.raises(ck.CheckpointError, match="no tensor"):
        st.get("backbone.layers.99.mixer.q_proj.weight")
    with pytest.raises(ck.CheckpointError, match="is U8, expected BF16"):
        st.get("backbone.layers.0.mixer.q_proj.weight", "BF16")
    with pytest.raises(ck.CheckpointError, match="has shape"):
        st.get("backbone.layers.0.mixer.q_proj.weight", "U8", (256, 64))
    data = open(os.path.join(ckpt_dir, "model.safetensors"), "rb").read()
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes((len(data) * 2).to_bytes(8, "little") + data[8:])
    with pytest.raises(ck.CheckpointError, match="bad header length"):
        ck.SafeTensors(str(bad))
    hlen = int.from_bytes(data[:8], "little")
    header = json.loads(data[8:8 + hlen])
    name = "backbone.layers.0.mixer.q_proj.weight"
    header[name]["data_offsets"][1] += 1 << 30
    hb = json.dumps(header).encode()
    bad.write_bytes(len(hb).to_bytes(8, "little") + hb + data[8 + hlen:])
    with pytest.raises(ck.CheckpointError, match="bad offsets"):
        ck.SafeTensors(str(bad))


@pytest.mark.parametrize("change,match", [
    ({"quantization_config": {"quant_algo": "FP8"}}, "W4A16_NVFP4"),
    ({"model_type": "llama"}, "not a Dory checkpoint"),
    ({"n_output_layers": 3}, "input \\+ recurrent \\+ output"),
    ({"layer_types": ["mlp"] * 8 + ["mlp"]}, "layer_types has 9"),
    ({"layer_types": ["conv"] * 8}, "unknown layer type"),
    ({"sliding_window": 0}, "sliding layers without a window"),
    ({"rope_parameters": {"full_attention": {"rope_theta": 1e6}}}, "no rope_theta"),
    ({"tie_word_embeddings": True}, "untied"),
])
def test_config_refusals(ck, ckpt_dir, tmp_path, change, match):
    c = json.load(open(os.path.join(ckpt_dir, "config.json")))
    c.update(change)
    d = tmp_path / "ck"
    d.mkdir()
    (d / "config.json").write_text(json.dumps(c))
    os.symlink(os.path.join(ckpt_dir, "model.safetensors"), str(d / "model.safetensors"))
    with pytest.raises(ck.CheckpointError, match=match):
        ck.DoryCheckpoint(str(d), context=1024)


def test_folded_vectors_and_layout(ck, ckpt_dir):
    c = ck.DoryCheckpoint(ckpt_dir, context=1024)
    cfg = c.cfg
    assert (cfg["hidden"], cfg["ffn"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["vocab"]) == \
        (256, 512, 4, 2, 64, 1000)
    assert (cfg["n_in"], cfg["n_rec"], cfg["n_out"], cfg["loops"], cfg["window"]) == (2, 4, 2, 2, 48)
    assert cfg["ring_slots"] == 48 + 16 and cfg["kv_dtype"] == ck.KV_FP8
    assert cfg["theta_sliding"] == 1e4 and cfg["theta_full"] == 1e6
    assert c.kinds == [ck.SLIDING, ck.MLP, ck.SLIDING, ck.MLP, ck.SLIDING, ck.MLP, ck.FULL, ck.MLP]
    tg = np.load(os.path.join(ckpt_dir, "folded_targets.npz"))
    np.testing.assert_allclose(c.logit_scale, tg["logit_scale"], rtol=8e-3)
    for i, L in enumerate(c.layers):
        for key in ("qscale", "gscale", "sg", "su", "lr"):
            if key in L:
                assert L[key].dtype == np.float32
                np.testing.assert_allclose(L[key], tg["%d.%s" % (i, key)], rtol=1.6e-2, err_msg="%d %s" % (i, key))
    codes, scales, glob = c.layers[0]["q"]
    st = c.st
    assert codes.ctypes.data == st.get("backbone.layers.0.mixer.q_proj.weight").ctypes.data   # a view, no copy
    assert scales.shape == (256, 16) and codes.shape == (256, 128)
    rows = c.embed([0, 999, 5])
    np.testing.assert_array_equal(rows.view(np.uint32) >> 16, c.embed_table[[0, 999, 5]].astype(np.uint32))
    with pytest.raises(ck.CheckpointError):
        c.embed([1000])

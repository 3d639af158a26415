"""A Dory checkpoint in ModelOpt's NVFP4 layout on the device (packs/dory/dory.cpp:316-364, 417-428): the
projections go from the mapped file to prepare() as they are (device repack), the BF16 LM head and the folded
vectors as the reference's constructor leaves them, FP8 caches (the pack's default); a prompt from the embedding
table in chunks, then steps, against the oracle holding the same checkpoint. Bars as the decode step's: logits
rel-L2 <= 1e-3 and the same argmax."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def rel_l2(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(np.asarray(y, np.float64) - ref) / np.linalg.norm(ref))


def test_checkpoint_prompt_and_steps(hip, pkg, orc, wl, ck, ckpt_dir):
    c = ck.DoryCheckpoint(ckpt_dir, context=512)
    tokens = np.random.default_rng(50).integers(0, c.cfg["vocab"], 140)
    x = c.embed(tokens)
    H, V = c.cfg["hidden"], c.cfg["vocab"]
    ref = orc.Dory(c, wl)
    want = np.concatenate([ref.forward(x[0:100], 0, threads=16)[-1:]] +
                          [ref.forward(x[p:p + 8], p) for p in range(100, 140, 8)])
    dev = hip.dory(c)
    dx = hip.array(x)
    dl = hip.array(shape=(8, V))
    got = []
    try:
        dev.prefill(dx, 100, 0, pkg.LOGITS_LAST, dl)
        got.append(dl.numpy()[:1])
        for p in range(100, 140, 8):
            dev.forward(dx.ptr + p * H * 4, 8, p, dl)
            got.append(dl.numpy())
    finally:
        dx.free()
        dl.free()
        dev.destroy()
    got = np.concatenate(got)
    e = rel_l2(got, want)
    print("checkpoint model, prompt of 100 then 5 steps of 8: logits rel-L2 %.2e" % e)
    assert e <= 1e-3
    assert (got.argmax(1) == want.argmax(1)).all()


def test_checkpoint_weights_repacked_from_the_map(hip, pkg, ck, ckpt_dir):
    """Every projection of the checkpoint prepared straight from the mapped file equals the documented tile layout
    of the same bytes."""
    from test_gpu_gemv import tiles_np
    c = ck.DoryCheckpoint(ckpt_dir, context=512)
    for L in c.layers:
        for name in ("q", "k", "v", "g", "o", "gate", "up", "down"):
            if name in L:
                w = pkg.Weight(*L[name])
                assert w.codes.ctypes.data == L[name][0].ctypes.data   # no copy on the host
                hip.prepare(w)
                got = hip.nvfp4_tiles(w)
                hip.release_weight(w)
                np.testing.assert_array_equal(got, tiles_np(L[name][0], L[name][1]))

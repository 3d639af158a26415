"""The oracle's Dory composition (oracle/oracle.c xo_dory_*, after packs/dory/dory.cpp:467-578) and the checkpoint
reader's folding of the scale vectors (xtier-go_amd/checkpoint.py, after dory.cpp:316-364) against the reference's own
CPU DorySession, compiled from its sources into oracle/_ref (oracle/Makefile) and run on synthetic ModelOpt
checkpoints (tests/make_checkpoint.py).

- The committed vectors (tests/golden/dory_*.npz) hold the reference session's logits over a schedule of a prompt
  chunk, 8-row verify steps, single steps past the sliding rings' wrap and a speculative rewind, for BF16 and FP8
  caches, per_loop and last_loop KV modes, one and two loops, heads of 64 and of 256 dims. The oracle must
  reproduce them to FP32 rounding (it follows the same operations in the same order: in practice bit for bit).
- Where oracle/_ref is built, the same comparison runs live on other tokens.
- Mistakes a restatement could plausibly make -- the gate scale folded without its square, the SwiGLU scales swapped,
  the MLP's negative alphas kept negative, the KV mode ignored -- each move the logits far beyond the bar.
- gate_norm and add_norm (dory.cpp:510-515, 530-541) against FP64 closed forms.
"""
import numpy as np
import pytest

import dory_golden as dg

BAR = 1e-6


@pytest.fixture(scope="module")
def ckroot(tmp_path_factory):
    return str(tmp_path_factory.mktemp("dory_golden_ckpt"))


def oracle_logits(orc, wl, c, g):
    model = orc.Dory(c, wl)
    return dg.run(lambda x, p: model.forward(x, p, threads=4), g, c.embed)


@pytest.mark.parametrize("name", dg.CASES)
def test_oracle_matches_reference_session(name, orc, wl, ck, ckroot):
    g = dg.load(name)
    d, sha = dg.checkpoint_dir(ckroot, g["variant"], int(g["seed"]))
    assert sha == g["sha256"], "tests/make_checkpoint.py no longer writes the checkpoint the vectors were made on"
    c = dg.open_checkpoint(ck, d, g["options"])
    rel, srel, same = dg.compare(oracle_logits(orc, wl, c, g), g)
    print("%s: rel-L2 %.2e, row norms %.2e, argmax %.3f" % (name, rel, srel, same))
    assert rel <= BAR and srel <= BAR and same == 1.0


@pytest.mark.parametrize("name", ["tiny_fp8_last_loop", "d256_bf16_per_loop"])
def test_oracle_matches_live_reference(name, orc, wl, ck, ckroot):
    if not orc.ref_available():
        pytest.skip("oracle/_ref is built only where the reference tree exists")
    g = dg.load(name)
    g["tokens"] = np.random.default_rng(4242).integers(0, 1000, len(g["tokens"])).astype(np.int32)
    d, _ = dg.checkpoint_dir(ckroot, g["variant"], int(g["seed"]))
    r = orc.RefDory(d, g["options"], threads=4)

    def ref_forward(tokens_of):
        out = []
        for pos0, off, n in g["schedule"]:
            if r.n_past != pos0:
                assert r.rewind(int(pos0))
            out.append(r.forward(g["tokens"][off:off + n]))
        return np.concatenate(out)

    want = ref_forward(None)
    r.close()
    c = dg.open_checkpoint(ck, d, g["options"])
    got = oracle_logits(orc, wl, c, g)
    rel = float(np.linalg.norm(got.astype(np.float64) - want) / np.linalg.norm(want.astype(np.float64)))
    assert rel <= BAR, rel
    assert (got.argmax(1) == want.argmax(1)).all()


def planted(kind, c, ck):
    """A plausible restatement mistake planted into the folded checkpoint (or its options)."""
    if kind == "gscale_unsquared":
        for L in c.layers:
            if "gscale" in L:
                L["gscale"] = np.sqrt(L["gscale"]).astype(np.float32)
    elif kind == "swiglu_scales_swapped":
        for L in c.layers:
            if "sg" in L:
                L["sg"], L["su"] = L["su"], L["sg"]
    elif kind == "alpha_sign_kept":
        for i, L in enumerate(c.layers):
            if "sg" in L:
                raw = c.vec("backbone.layers.%d.mlp_alpha" % i, c.cfg["hidden"])
                L["lr"] = (raw * np.float32(0.05 / 0.02)).astype(np.float32)
    elif kind == "kv_mode_ignored":
        c.cfg["kv_mode"] = 1 - c.cfg["kv_mode"]
    return c


@pytest.mark.parametrize("kind", ["gscale_unsquared", "swiglu_scales_swapped", "alpha_sign_kept", "kv_mode_ignored"])
def test_planted_mistakes_fail_the_vectors(kind, orc, wl, ck, ckroot):
    g = dg.load("tiny_fp8_last_loop")
    d, _ = dg.checkpoint_dir(ckroot, g["variant"], int(g["seed"]))
    c = planted(kind, dg.open_checkpoint(ck, d, g["options"]), ck)
    rel, _, _ = dg.compare(oracle_logits(orc, wl, c, g), g)
    print("%s: rel-L2 %.2e" % (kind, rel))
    assert rel > 1e3 * BAR


# --- the attention gate and the loop norms against FP64 ---

def justnorm64(x):
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + 1e-6)


def test_gate_norm_closed_form(orc):
    """att * sigmoid(g * gs), then justnorm over the row (dory.cpp:510-515)."""
    rng = np.random.default_rng(61)
    att = rng.standard_normal((3, 4096)).astype(np.float32)
    gate = (rng.standard_normal((3, 4096)) * 3).astype(np.float32)
    gs = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    got = orc.gate_norm(att, gate, gs)
    want = justnorm64(att * (1 / (1 + np.exp(-gate.astype(np.float64) * gs))))
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < 1e-5, err
    # planted in the closed form: the gate's sign flipped, the scale left out, no norm
    for wrong in (justnorm64(att * (1 / (1 + np.exp(gate.astype(np.float64) * gs)))),
                  justnorm64(att * (1 / (1 + np.exp(-gate.astype(np.float64)))))):
        assert np.abs(got - wrong).max() / np.abs(want).max() > 1e-2
    assert np.abs(got - att * (1 / (1 + np.exp(-gate.astype(np.float64) * gs)))).max() > 1e-2


def test_add_norm_closed_form(orc):
    """The loop entry justnorm(state + input) and exit justnorm(x) (dory.cpp:530-541)."""
    rng = np.random.default_rng(62)
    a = rng.standard_normal((4, 3072)).astype(np.float32)
    b = rng.standard_normal((4, 3072)).astype(np.float32)
    err = np.abs(orc.add_norm(a, b) - justnorm64(a.astype(np.float64) + b)).max()
    assert err < 1e-6, err
    err = np.abs(orc.add_norm(a) - justnorm64(a)).max()
    assert err < 1e-6, err
    assert np.abs(orc.add_norm(a, b) - justnorm64(a)).max() > 1e-3   # the input left out
    # the first loop's entry justnorm(x + x) keeps x's direction
    x = justnorm64(a).astype(np.float32)
    assert np.abs(orc.add_norm(x, x) - x).max() < 1e-6

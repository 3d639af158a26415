"""The HIP Dory session (xtg_hip_dory_create / forward through the C ABI) against the reference's own CPU
DorySession (packs/dory/dory.cpp:304-578): the committed vectors of tests/golden/dory_*.npz, made by the reference
compiled from its sources, replayed on the same synthetic ModelOpt checkpoints (tests/make_checkpoint.py, checked by
sha256). The device reads the checkpoint as the reference does (NVFP4 projections from the mapped file, BF16 LM head,
folded vectors), and runs the schedule's calls: a 30-row prompt chunk (the prefill kernels), 8-row verify steps and
single steps (the fused decode kernels) past the 64-slot rings' wrap, and 8 drafts of which 3 are kept (the next
call starts at the rewound position). Cases: BF16 and FP8 caches, per_loop and last_loop KV modes, one and two loops,
heads of 64 and 256 dims. Bar (the north star's): logits rel-L2 <= 1e-3 and the same argmax on every row."""
import numpy as np
import pytest

import dory_golden as dg

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ckroot(tmp_path_factory):
    return str(tmp_path_factory.mktemp("dory_golden_ckpt"))


@pytest.mark.parametrize("name", dg.CASES)
def test_device_session_matches_reference_session(name, hip, ck, ckroot):
    g = dg.load(name)
    d, sha = dg.checkpoint_dir(ckroot, g["variant"], int(g["seed"]))
    assert sha == g["sha256"], "tests/make_checkpoint.py no longer writes the checkpoint the vectors were made on"
    c = dg.open_checkpoint(ck, d, g["options"])
    H, V = c.cfg["hidden"], c.cfg["vocab"]
    most = int(max(n for _, _, n in g["schedule"]))
    dev = hip.dory(c)
    dx = hip.array(shape=(most, H))
    dl = hip.array(shape=(most, V))

    def forward(x, pos0):
        n = x.shape[0]
        hip.write(dx.ptr, np.ascontiguousarray(x, np.float32))
        dev.forward(dx, n, pos0, dl)
        return dl.numpy()[:n].copy()

    try:
        logits = dg.run(forward, g, c.embed)
    finally:
        dx.free()
        dl.free()
        dev.destroy()
    rel, srel, same = dg.compare(logits, g)
    print("%s: logits rel-L2 %.2e (row norms %.2e), argmax %.3f" % (name, rel, srel, same))
    assert rel <= 1e-3 and srel <= 1e-3
    assert same == 1.0

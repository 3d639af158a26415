"""The Dory golden vectors of the reference's own CPU session (tests/golden/dory_*.npz, written by
tests/golden/make_golden.py from packs/dory/dory.cpp compiled into oracle/_ref) and the means to replay their schedule
on another implementation: the checkpoint they were made on is rebuilt by tests/make_checkpoint.py (checked against
the sha256 kept with the vectors), read by xtier-go_amd/checkpoint.py with the case's launch options, and each
schedule entry (pos0, token offset, n) is one forward call of n rows at positions pos0 .. with the embedding rows of
those tokens."""
import hashlib
import json
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
CASES = sorted(f[len("dory_"):-len(".npz")] for f in os.listdir(GOLDEN) if f.startswith("dory_") and f.endswith(".npz"))
KV_DTYPES = {"bf16": 0, "fp8": 1}


def load(name):
    z = np.load(os.path.join(GOLDEN, "dory_%s.npz" % name))
    g = {k: z[k] for k in z.files}
    g["variant"] = str(g["variant"])
    g["sha256"] = str(g["sha256"])
    g["options"] = json.loads(str(g["options"]))
    return g


def checkpoint_dir(root, variant, seed):
    """The case's checkpoint, written once per (variant, seed) under root; returns (dir, sha256 of its safetensors)."""
    d = os.path.join(root, "%s_%d" % (variant, seed))
    if not os.path.exists(os.path.join(d, "model.safetensors")):
        subprocess.run([sys.executable, os.path.join(HERE, "make_checkpoint.py"), d, str(seed), variant], check=True)
    with open(os.path.join(d, "model.safetensors"), "rb") as f:
        return d, hashlib.sha256(f.read()).hexdigest()


def open_checkpoint(ck, d, options):
    """DoryCheckpoint with the pack options of a case (dory.cpp:136-170; the defaults are the checkpoint's)."""
    return ck.DoryCheckpoint(d, context=int(options.get("context", 32768)),
                             kv_dtype=KV_DTYPES[options.get("kv_dtype", "fp8")], loops=options.get("loops"),
                             kv_mode=options.get("kv_mode"))


def run(forward, g, embed):
    """Replays the case's schedule through forward(x_rows, pos0) -> logits [n][vocab]; all rows, concatenated."""
    out = []
    for pos0, off, n in g["schedule"]:
        out.append(forward(embed(g["tokens"][off:off + n]), int(pos0)))
    return np.concatenate(out)


def compare(logits, g):
    """(rel-L2 over the kept rows, largest row rel-L2 of the sums' check, argmax agreement) against the vectors."""
    kept = np.asarray(logits, np.float64)[g["rows"]]
    ref = g["logits"].astype(np.float64)
    rel = float(np.linalg.norm(kept - ref) / np.linalg.norm(ref))
    l64 = np.asarray(logits, np.float64)
    sumsq_rel = float(np.max(np.abs(np.sqrt((l64 * l64).sum(1)) - np.sqrt(g["sumsq"])) / np.sqrt(g["sumsq"])))
    same = float((np.asarray(logits).argmax(1) == g["argmax"]).mean())
    return rel, sumsq_rel, same

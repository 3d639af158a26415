"""Builds libxtg_hip.so (the gfx950 kernel layer behind include/xtg_hip.h) in-tree with hipcc.

Every source in csrc/ is compiled for gfx950 only, with packed-FP32 instructions disabled; objects go to
_build/ next to this file and the library to libxtg_hip.so beside it. `build.py --stamps` builds the phase-stamp
variant instead (-DXTG_PHASE_STAMPS: the GEMV's waves record when each phase of theirs ends; objects in
_build/stamps/, library libxtg_hip_stamps.so), which `bench.py --gemv-phases` loads; the product never does.
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libxtg_hip.so")
STAMPS_LIB = os.path.join(HERE, "libxtg_hip_stamps.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _compile(src, stamps=False):
    obj = os.path.join(OBJ, "stamps" if stamps else "", os.path.basename(src) + ".o")
    cmd = [HIPCC] + FLAGS + (["-DXTG_PHASE_STAMPS"] if stamps else []) + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the packed-FP32 feature and says so: not an error
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed on %s:\n%s" % (src, msg))
    return obj, msg


def build(verbose=False, stamps=False):
    os.makedirs(os.path.join(OBJ, "stamps") if stamps else OBJ, exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        results = list(ex.map(lambda src: _compile(src, stamps), srcs))
    for obj, msg in results:
        if verbose and msg.strip():
            print(msg, file=sys.stderr)
    lib = STAMPS_LIB if stamps else LIB
    tmp = lib + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + [o for o, _ in results]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    print(build(verbose=True, stamps="--stamps" in sys.argv[1:]))

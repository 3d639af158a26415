"""The C-ABI library loads without a GPU and exports every entry point include/*.h declares; the Python binding
declares a signature for each; no compute call is made here."""
import ctypes
import glob
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(xtg_hip_\w+)\s*\(", text))
    return names


def test_header_declares_entry_points():
    names = declared_functions()
    assert {"xtg_hip_open", "xtg_hip_close", "xtg_hip_matmul_nvfp4", "xtg_hip_matmul_nvfp4_dev"} <= names


def test_library_exports_every_declared_symbol(pkg):
    lib = ctypes.CDLL(pkg.LIB_PATH)
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_header(pkg):
    bound = {name for name, _, _ in pkg.SIGNATURES}
    assert declared_functions() == bound


def test_struct_layout_matches_reference_weight(pkg):
    # xtg::Nvfp4Weight: two pointers, a float, two ints (engine/include/xtg/kernels.h:13-20)
    assert ctypes.sizeof(pkg.Nvfp4) == 8 + 8 + 4 + 4 + 4 + 4   # trailing padding to 8
    assert pkg.Nvfp4.glob.offset == 16 and pkg.Nvfp4.n_out.offset == 20 and pkg.Nvfp4.k.offset == 24

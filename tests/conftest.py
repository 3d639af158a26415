import importlib.util
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libxtg_hip.so")
    # the CPU oracle is test infrastructure built from oracle/oracle.c; build it when it is missing
    if not os.path.exists(os.path.join(ROOT, "oracle", "liboracle.so")):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "all"], check=True)


def load_package():
    """The xtier-go_amd package (its directory name is not an identifier, so it is loaded by path)."""
    if "xtier_go_amd" in sys.modules:
        return sys.modules["xtier_go_amd"]
    pkg_dir = os.path.join(ROOT, "xtier-go_amd")
    spec = importlib.util.spec_from_file_location("xtier_go_amd", os.path.join(pkg_dir, "__init__.py"),
                                                  submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["xtier_go_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def pkg():
    return load_package()


@pytest.fixture(scope="session")
def wl():
    load_package()
    import xtier_go_amd.workloads as w
    return w


@pytest.fixture(scope="session")
def orc():
    import oracle as o
    return o


@pytest.fixture(scope="session")
def hip(pkg):
    """One backend for the whole GPU session (one process, one device)."""
    b = pkg.HipBackend(0)
    yield b
    b.close()


@pytest.fixture(scope="session")
def ck():
    """The checkpoint reader (xtier-go_amd/checkpoint.py)."""
    load_package()
    import xtier_go_amd.checkpoint as c
    return c


@pytest.fixture(scope="session")
def ckpt_dir(tmp_path_factory):
    """A small Dory checkpoint in ModelOpt's NVFP4 layout, written by the safetensors library in a process of its own
    (tests/make_checkpoint.py)."""
    d = str(tmp_path_factory.mktemp("dory_ckpt"))
    subprocess.run([sys.executable, os.path.join(ROOT, "tests", "make_checkpoint.py"), d, "3"], check=True)
    return d

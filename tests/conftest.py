"""pytest configuration: the `gpu` marker, import paths and shared fixtures.

CPU tests (`-m "not gpu"`) cover the oracle against the reference's own vectors and the
mathematics, the host planner and argument validation, the C ABI exports and the Node engine.
GPU tests (`-m gpu`) call libqattn.so through its C ABI on a gfx950 device and compare with the
oracle on identical inputs.
"""
import importlib.util
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "qwen3-embedding-webgpu-prepacked_amd")
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, os.path.join(REPO, "tests"))


def load_qattn():
    """Import the package's ctypes binding (the package directory name has dashes)."""
    if "qattn" in sys.modules:
        return sys.modules["qattn"]
    spec = importlib.util.spec_from_file_location("qattn", os.path.join(PKG, "qattn.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["qattn"] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X); runs through libqattn.so")


@pytest.fixture(scope="session")
def qattn():
    return load_qattn()


@pytest.fixture(scope="session")
def oracle():
    import oracle as orc
    if not os.path.exists(orc.LIB_PATH):
        orc.build()
    return orc


@pytest.fixture(scope="session")
def ctx(qattn):
    c = qattn.Context(0)
    yield c
    c.close()

"""Shared fixtures: the product package (loaded from qwen3-iree_amd/) and the
CPU oracle (oracle/, the checker)."""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
PKG_DIR = REPO / "qwen3-iree_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the C ABI")


def _load_package():
    name = "qwen3_iree_amd"
    if name not in sys.modules:
        spec = importlib.util.spec_from_file_location(
            name, PKG_DIR / "__init__.py", submodule_search_locations=[str(PKG_DIR)])
        mod = importlib.util.module_from_spec(spec)
        sys.modules[name] = mod
        spec.loader.exec_module(mod)
    return sys.modules[name]


_load_package()
sys.path.insert(0, str(REPO / "oracle"))


@pytest.fixture(scope="session")
def O():
    import oracle

    if not oracle.LIB_PATH.exists():
        oracle.build()
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def Q():
    from qwen3_iree_amd import q8gemv

    q8gemv.load_library()
    return q8gemv


@pytest.fixture(scope="session")
def Wt():
    from qwen3_iree_amd import weights

    return weights


@pytest.fixture(scope="session")
def gpu(Q):
    """Initialised library on device 0.  Fails (never skips) when the code
    object cannot be loaded: GPU tests must run the HIP path."""
    Q.init()
    return Q


@pytest.fixture(scope="session")
def model_host():
    """Seeded random-init Qwen3-0.6B parameters in the device layout (~1.1 GB)."""
    from qwen3_iree_amd import decode

    return decode.synthetic_weights(seed=0)

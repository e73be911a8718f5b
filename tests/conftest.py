import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built liblarder_moe.so")


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this process")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def built_lib():
    """The in-tree library, built here when it is missing (hipcc cross-compiles gfx950 without a GPU)."""
    from larder_amd import _lib
    if not _lib.LIB_PATH.exists():
        from larder_amd import build
        build.build()
    return _lib.lib()


@pytest.fixture(scope="session")
def rng_seed():
    return int(os.environ.get("LMOE_TEST_SEED", "0"))

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (str(ROOT), str(ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device and the built library")
    config.addinivalue_line("markers", "slow: long-running (full-size configs)")


def _gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no HIP device visible (GPU tests run on the MI355X box)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle_lib():
    """Builds (if needed) and loads the C oracle."""
    from oracle import cscan

    cscan._load()
    return cscan


@pytest.fixture(scope="session")
def dev():
    import torch

    from mamba_metal_amd import _lib

    _lib.load()  # the HIP library must be there on a GPU box: fail loudly otherwise
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before any GPU work so a fault on the box is attributable.
    if "gpu" in request.keywords:
        print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
    yield

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "rumik-fast_amd"
# the reference engine puts its kernels/ directory on sys.path and imports cuda_gemv, mm_int4, ... by name;
# the tests use the drop-in modules the same way
for p in (PKG / "kernels", PKG / "engine", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def _gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible (GPU tests run on the MI355X box)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def dev():
    import torch
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _announce(request):
    # name the case before any GPU work, so a run that dies still says which test it was in
    if "gpu" in request.keywords:
        print(f"\n[gpu-test] {request.node.nodeid}", flush=True)
    yield

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG_ROOT = REPO / "taomate-hd_amd"
for p in (str(REPO), str(PKG_ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libtmhd.so")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def torch_mod():
    import torch

    return torch


@pytest.fixture(scope="session")
def dev(torch_mod):
    from taomate_hd_amd import _native

    _native.load()  # fail loudly if the HIP library is missing where a GPU is present
    return torch_mod.device("cuda:0")


def pytest_runtest_setup(item):
    # name the case before any GPU work, so a lost box still says what ran
    if "gpu" in item.keywords:
        sys.stdout.write(f"\n[gpu-case] {item.nodeid}\n")
        sys.stdout.flush()

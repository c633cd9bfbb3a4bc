import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built library")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this process")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def lib():
    """The loaded kernel library (built by __graft_entry__.build() beforehand)."""
    from claudemaxing_amd import _lib

    return _lib.load()


@pytest.fixture(scope="session")
def dev():
    import torch

    return torch.device("cuda", 0)


def banner(msg):
    """Name the case on stdout before a GPU step, so a fatal failure still says which one."""
    print(f"[case] {msg}", flush=True)
    os.sys.stdout.flush()

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))

LIBRARY = ROOT / "synapse_amd" / "_lib" / "libsynapse_kv.so"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library on cuda:0)")


def _ensure_library():
    # Tests load what __graft_entry__.build() produced; build only when nothing is there.
    if not LIBRARY.exists():
        from synapse_amd.build import build_library

        build_library()


@pytest.fixture(scope="session")
def native():
    _ensure_library()
    from synapse_amd.native import NativeKvLibrary

    return NativeKvLibrary.load()


@pytest.fixture(scope="session")
def torch_gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("the gpu tests need a HIP device (torch.cuda.is_available() is False)")
    return torch

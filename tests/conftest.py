"""Shared pytest setup: the `gpu` marker, import paths for the package and the oracle, seeded RNG helpers."""
import os
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
PKG_DIR = ROOT / "omarchy-mac-torch_amd"
for p in (str(ROOT), str(PKG_DIR)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libomt_hip.so on cuda:0)")


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def cuda():
    """The GPU parity tests run only on a box with a GPU; elsewhere they are an error, not a silent skip."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return torch.device("cuda:0")

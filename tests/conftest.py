"""Shared pytest setup: the `gpu` marker, the package loader and the oracle."""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(Path(__file__).resolve().parent))

from helpers import load_pkg, load_oracle, gpu_available  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels")


@pytest.fixture(scope="session")
def mcv():
    return load_pkg()


@pytest.fixture(scope="session")
def oracle():
    return load_oracle()


@pytest.fixture(scope="session")
def cuda():
    if not gpu_available():
        pytest.skip("no GPU in this environment")
    import torch
    return torch.device("cuda:0")

"""Test configuration: `gpu` marker, import paths for the package and the
CPU oracle, and session fixtures."""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "mamb2_8b_fp4_recall_sq3.25_amd"
for p in (str(ROOT), str(PKG), str(ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.build()
    return o


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def model(device):
    """A random-init Mamba-2 8B model of the real geometry on the GPU (built
    once per session; tests may overwrite its projection weights)."""
    import torch
    from mamba2_model import random_model
    print("[model] building the random 8B model", flush=True)
    m = random_model(device)
    torch.cuda.synchronize()
    return m

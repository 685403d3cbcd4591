"""Shared test setup.

Markers: ``gpu`` = needs an MI355X (run with ``-m gpu`` on the GPU box);
everything else runs on the CPU (oracle pinning, host logic, ABI surface).
"""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "ops-gnn_amd", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

SEED = 42


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test needs an AMD MI355X GPU")


@pytest.fixture(scope="session")
def ogn():
    """The ops_gnn package on a GPU box (fails loudly if the HIP library is missing)."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    import ops_gnn

    return ops_gnn


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o

    return o

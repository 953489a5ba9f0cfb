"""pytest configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs the oracle pins, host-side logic and the C-ABI symbol
check on CPU; ``-m gpu`` runs the HIP parity tests (a ROCm device is required).
"""

from __future__ import annotations

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(REPO, "kda-csa-hca-fusion_amd")
for _p in (PKG_DIR, REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libkch.so")
    config.addinivalue_line("markers", "slow: larger CPU oracle cases")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda:0")

"""Test configuration: the ``gpu`` marker and shared fixtures.

``-m "not gpu"`` runs on any host (oracle vs golden vectors and closed forms,
byte encoding, library exports).  ``-m gpu`` needs an MI355X and compares
libane_amd.so against the CPU oracle through the C ABI.
"""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libane_amd.so")


@pytest.fixture(scope="session")
def oracle():
    from tests import _oracle

    return _oracle.load()


@pytest.fixture(scope="session")
def ane():
    """The product library; GPU tests fail (not skip) when it is unusable."""
    import torch

    import ane_amd

    assert torch.cuda.is_available(), "GPU test selected but torch sees no GPU"
    ane_amd.require_gpu()
    return ane_amd

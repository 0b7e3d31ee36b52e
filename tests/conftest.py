"""Shared pytest setup.

* Registers the ``gpu`` marker: tests that need an MI355X (ROCm device) and
  the built ``libsk_attn.so``.  ``pytest -m "not gpu"`` runs everywhere.
* Puts the repository root on ``sys.path`` so ``stackkernels_amd`` and the
  ``oracle`` (test infrastructure) import without installation.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


@pytest.fixture
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda:0")

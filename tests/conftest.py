"""Test configuration: the ``gpu`` marker, and the repository root on the import path.

``-m "not gpu"`` runs here without a GPU: the oracle against its pins, the host logic, and the
C-ABI library's exports. ``-m gpu`` runs on an MI355X: the HIP path against the oracle.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def ext():
    """The loaded kernels; a GPU test fails (never skips) when they cannot load."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a GPU")
    from everserve_amd import kernels

    return kernels.load()

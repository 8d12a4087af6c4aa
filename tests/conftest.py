"""Test configuration: import paths and the ``gpu`` marker.

CPU tests (``-m "not gpu"``) cover the oracle against closed forms and known
answers, the host-side API contract and the C ABI surface.  GPU tests
(``-m gpu``) compare the HIP kernels, called through the C ABI, with the
oracle on seeded inputs.
"""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG_ROOT = ROOT / "neuronmlp-on-tpu_amd"
for p in (str(ROOT), str(PKG_ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: full-size shapes")


@pytest.fixture(scope="session")
def gpu():
    """The HIP library on cuda:0.  Skips only when no GPU is visible at all;
    on a GPU box a missing library is an error, not a skip."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import svdmlp

    svdmlp.load()
    return torch.device("cuda:0")

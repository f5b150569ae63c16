"""Test configuration: the ``gpu`` marker and shared fixtures.

Two tiers, as in the reference (tests/conftest.py:8-26 skips GPU files
without a Metal device):

* ``-m "not gpu"`` - oracle against golden vectors and closed forms, host
  logic, C-ABI loading and argument validation.  Runs without a GPU.
* ``-m gpu`` - parity of the HIP kernels against the oracle on an MI355X,
  through the C ABI.  A GPU test on a host without a GPU FAILS (it is never
  silently skipped), so a GPU run that lost its device cannot pass.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libneso_amd.so")


@pytest.fixture(scope="session")
def golden_dir() -> Path:
    return GOLDEN


@pytest.fixture(scope="session")
def gpu():
    """The cuda:0 device; fails the test when no GPU is visible."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected but torch.cuda.is_available() is False")
    name = torch.cuda.get_device_properties(0).gcnArchName
    if not name.startswith("gfx950"):
        pytest.fail(f"expected a gfx950 device, found {name}")
    import neso_amd._lib as lib

    lib.load()
    return torch.device("cuda:0")

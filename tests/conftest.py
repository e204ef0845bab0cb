"""pytest configuration: markers and shared fixtures.

Markers
  gpu        needs an MI355X (run with -m gpu on the GPU box)
  extensive  larger sweeps (deselect with -m "not extensive")
"""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test needs an MI355X GPU")
    config.addinivalue_line("markers", "extensive: extensive test suite")
    # operators' reference() in the tests is the CPU oracle
    from iron_amd.common import set_reference_provider

    from tests import oracle_provider

    set_reference_provider(oracle_provider.reference)


@pytest.fixture(scope="session")
def gpu():
    """torch.device('cuda', 0) with libiron_hip loaded; skips without a GPU."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from iron_amd import _lib

    _lib.load()  # raises if the HIP library is not built: never a silent fallback
    return torch.device("cuda", 0)

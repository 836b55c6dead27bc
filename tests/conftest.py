"""Pytest configuration: the ``gpu`` marker and shared import paths.

Tests marked ``gpu`` need a ROCm GPU (MI355X) and the built ``libgdn2_hip.so``;
everything else runs on the CPU.  ``oracle/`` is importable from tests only.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running test")


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test selected but no ROCm GPU is visible")
    return torch.device("cuda", 0)

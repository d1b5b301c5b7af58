"""Pytest configuration: the `gpu` marker and shared fixtures.

GPU tests call libc3hip.so kernels on an MI355X and compare with the NumPy
oracle under oracle/; CPU tests check the oracle, the planner and the ABI.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libc3hip.so")


@pytest.fixture(scope="session")
def gpu():
    """Initialise device 0 through libc3hip.so; fail loudly if it is missing."""
    from hackathon_amd import device

    device.init(0)
    return device

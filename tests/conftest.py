"""Shared test setup: import paths, the `gpu` marker and common fixtures.

Tests marked `gpu` need an MI355X and call the HIP library through its C ABI;
every other test runs on the CPU (oracle pins, host logic, library exports).
"""

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "needle.js_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and libneedle_hip.so")


@pytest.fixture(scope="session")
def hip():
    """One HipBackend for the GPU session (fails loudly without a device)."""
    from needle_hip import HipBackend

    backend = HipBackend()
    yield backend
    backend.dispose()


@pytest.fixture
def rng():
    return np.random.default_rng(1234)

"""pytest configuration: the `gpu` marker and shared helpers.

Tests marked ``gpu`` need a real MI355X and call the HIP library through its
C ABI; everything else runs on the CPU (oracle pinning, host logic, library
symbol checks)."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X / gfx950)")


@pytest.fixture(scope="session", autouse=True)
def _oracle_built():
    import oracle

    if not os.path.exists(oracle._LIB_PATH):
        oracle.build()
    yield

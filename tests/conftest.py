"""Shared test set-up: the `gpu` marker, import paths and the device session."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; calls libingot_rocm.so through its C ABI")


@pytest.fixture(scope="session")
def sess():
    """One library session on device 0 for the whole GPU run."""
    from ingot_amd import Session

    s = Session(0)
    yield s
    s.close()

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


@pytest.fixture
def env_session(monkeypatch):
    """Opens extra library sessions with INGOT_* test hooks set (INGOT_GEMM_CFG, INGOT_GEMV_CFG, INGOT_I8G_ROWS,
    INGOT_NO_GEMV, INGOT_QCONV_PATH): a session reads them once, when it opens."""
    from ingot_amd import Session

    opened = []

    def open_with(**env):
        for k, v in env.items():
            monkeypatch.setenv(k, str(v))
        s = Session(0)
        opened.append(s)
        return s

    yield open_with
    for s in opened:
        s.close()

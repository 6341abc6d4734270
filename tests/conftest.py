"""Shared test setup: import paths, the `gpu` marker, the device fixture."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "lightx2v-rs_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


@pytest.fixture(scope="session")
def be():
    """One HipBackend for the GPU tests.  Skips only where no HIP device is
    visible at all (a CPU host); on a GPU host a failed create is an error."""
    import lightx2v_hip as H

    if H.device_count() == 0:
        pytest.skip("no HIP device visible")
    b = H.HipBackend(0)
    yield b
    b.close()

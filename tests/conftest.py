import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "birdnet-neon-engine_amd")
for p in (PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) and libbnneon_hip.so")


@pytest.fixture(scope="session")
def hip():
    """The kernel-level binding, with a visible GPU (fails loudly otherwise)."""
    from bnneon import hip as H
    n = H.lib().bnh_device_count()
    assert n > 0, "no HIP device visible: the gpu tests need an MI355X"
    return H

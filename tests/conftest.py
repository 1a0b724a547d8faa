import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "rust-ts-tokio-inference-engine_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path through the C-ABI)")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def bridge():
    """The product library on a GPU; fails loudly if it is missing."""
    import hip_bridge

    lib = hip_bridge.load()
    if lib.hb_device_count() < 1:
        pytest.fail("no HIP device visible to libhip_bridge")
    return hip_bridge

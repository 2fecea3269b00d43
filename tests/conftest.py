"""pytest configuration: the `gpu` marker, import paths and shared fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "-damn-low-level-fence-inference-version-1_amd")
TESTS = os.path.dirname(os.path.abspath(__file__))
for p in (TESTS, PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(autouse=True)
def _release_device_inputs():
    yield
    import gpu_util
    gpu_util.LIVE.clear()


@pytest.fixture(scope="session")
def oracle():
    from oracle_py import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def fence():
    import fence_ops
    fence_ops.lib()
    return fence_ops

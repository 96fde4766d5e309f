"""pytest configuration: the `gpu` marker, import paths and shared fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "wzy-flash-serve_amd")
for p in (PKG, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu on the GPU box)")


@pytest.fixture(scope="session")
def wz():
    import wzy_amd
    return wzy_amd.lib()


@pytest.fixture(scope="session")
def orc():
    import oracle_lib
    return oracle_lib.load()


@pytest.fixture(scope="session")
def gpu(wz):
    """Device 0 through libwzy_amd (GPU tests never import torch: one HIP runtime per process)."""
    import wzy_amd
    if wzy_amd.device_count() < 1:
        pytest.fail("GPU test collected but no GPU is visible")
    wz.wzy_dev_set(0)
    return 0

"""Shared pytest setup: the `gpu` marker, import paths, the backend handle."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) and the built HIP backend")


@pytest.fixture(scope="session")
def dsv4():
    """The binding module of deepseek-v4-in-c_amd/ (imported by path: the
    directory name is not a Python identifier)."""
    import common
    return common.load_pkg()


@pytest.fixture(scope="session")
def gpu(dsv4):
    """An initialised backend. A GPU test run without a device fails loudly:
    there is no CPU fallback to skip to."""
    L = dsv4.lib()
    if not L.dsv4_gpu_available():
        pytest.fail("no HIP device visible: GPU tests need an MI355X")
    assert L.dsv4_gpu_init() == 0
    return L

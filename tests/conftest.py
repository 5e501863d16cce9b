"""pytest configuration: the `gpu` marker and shared fixtures.

Tests marked `gpu` need an MI355X (gfx950) and the in-tree libraries; they run
with `pytest -m gpu` on the GPU box. Everything else runs on the CPU.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libraries")


@pytest.fixture(scope="session")
def libs():
    import grxcp_amd
    return grxcp_amd.load()


@pytest.fixture(scope="session")
def gpu(libs):
    """The GPU session: device 0 selected, a gfx950 required (no skip: a GPU
    test that cannot find its device must fail, not pass silently)."""
    import grxcp_amd
    n = grxcp_amd.device_count()
    assert n > 0, "no HIP device visible to a gpu-marked test"
    grxcp_amd.check_rt(libs.rt.grxSetDevice(0), "grxSetDevice")
    return libs


@pytest.fixture()
def blas(gpu):
    import grxcp_amd
    b = grxcp_amd.Blas()
    yield b
    b.close()


@pytest.fixture()
def dnn(gpu):
    import grxcp_amd
    d = grxcp_amd.Dnn()
    yield d
    d.close()

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libgolem_hip.so")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.load()
    return oracle


@pytest.fixture(scope="session")
def dev():
    """The GPU tests' device helper: a gx context on cuda:0, with torch as the
    allocator of device buffers."""
    from tests.gpu_util import Device
    d = Device()
    yield d
    d.close()

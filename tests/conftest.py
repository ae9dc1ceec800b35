import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and libdpuf_amd.so")


@pytest.fixture(scope="session")
def tools():
    from dpuf_amd import abi
    return abi.load_tools()


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as O
    return O.load()


@pytest.fixture(scope="session")
def eng():
    from dpuf_amd import abi
    lib = abi.load_engine()
    if not lib.dpuf_amd_device_ok():
        raise RuntimeError("GPU test started without a visible HIP device")
    return lib

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import pko
    pko.lib()
    return pko


@pytest.fixture(scope="session")
def abi():
    import parakeet_wgsl_amd.palette_abi as abi
    abi.load()
    return abi


@pytest.fixture(scope="session")
def workloads():
    import parakeet_wgsl_amd.workloads as wl
    return wl


@pytest.fixture(scope="session")
def ctx(abi):
    context = abi.Context(0)
    info = context.info()
    arch = info.arch.decode()
    if not arch.startswith("gfx950"):
        pytest.fail(f"expected a gfx950 device, found {arch}")
    yield context
    context.close()

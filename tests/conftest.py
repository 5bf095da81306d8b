import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")
    config.addinivalue_line("markers", "slow: longer CPU-only case")


@pytest.fixture(scope="session")
def olib():
    import oracle_lib
    return oracle_lib.lib()


@pytest.fixture(scope="session")
def rlib():
    import oracle_lib
    r = oracle_lib.ref()
    if r is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    return r

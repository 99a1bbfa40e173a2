import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libkt_gfx950.so")
    config.addinivalue_line("markers", "slow: full-size shapes")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle

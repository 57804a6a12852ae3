import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def oracle():
    from oracle import build as ob
    from oracle import moe_oracle as O
    if not os.path.exists(ob.OUT):
        ob.build()
    O.lib()
    return O

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "aot-llm_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libaotk.so)")


@pytest.fixture(scope="session")
def aotk():
    import aotk as A
    A.init(0)
    return A


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.load()
    return O

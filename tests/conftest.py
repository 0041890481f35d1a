import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs libllmk's HIP kernels)")


@pytest.fixture(scope="session")
def llmk():
    from __graft_entry__ import load_llmk
    return load_llmk()


@pytest.fixture(scope="session")
def orc():
    import oracle
    return oracle

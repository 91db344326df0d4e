import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "qwen3-vl-2b-inference_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def orc():
    from checkers import Oracle
    return Oracle.load()


@pytest.fixture(scope="session")
def ref():
    from checkers import Reference
    r = Reference.load()
    if r is None:
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    return r

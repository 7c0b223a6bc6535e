import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "gemma4-js_amd")
for p in (os.path.join(ROOT, "oracle"), PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libg4hip.so")


@pytest.fixture(scope="session")
def g4():
    """libg4hip initialised on device 0 (GPU tests only; fails loudly without it)."""
    import g4hip
    g4hip.init(0)
    return g4hip


@pytest.fixture(scope="session")
def oracle():
    import g4oracle
    g4oracle.lib()
    return g4oracle

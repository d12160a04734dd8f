import os
import sys

import pytest

try:  # import once at collection: the first import on a fresh box is slow
    import torch  # noqa: F401
except Exception:  # CPU-only environments without torch still run the oracle tests
    torch = None

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the libkmoe C ABI")


@pytest.fixture(scope="session")
def orc():
    from oracle import pyoracle

    pyoracle.lib()
    return pyoracle

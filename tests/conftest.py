import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "skyla-kernel_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libskyla_hip.so")


@pytest.fixture(scope="session")
def ctx():
    """One backend context for every GPU test (no fallback: fails without a device)."""
    from skyla_hip import Context

    c = Context.new(0)
    yield c
    c.free()

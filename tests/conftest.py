import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "xlstm-metal_amd")
for p in (ROOT, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    # GPU tests print the case they run before each GPU step (see gpu_case).
    pass


@pytest.fixture
def gpu_case(request):
    """Print and flush the test id before any GPU work, so a fault names its case."""
    print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
    return request.node.nodeid

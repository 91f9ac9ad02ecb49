import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(autouse=True)
def _announce(request):
    # name the case before it runs, so a GPU failure can be attributed
    print(f"\n[case] {request.node.nodeid}", flush=True)
    yield

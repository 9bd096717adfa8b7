import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


@pytest.fixture(scope="session")
def hip():
    """The HIP C-ABI, initialised on device 0 (GPU tests only)."""
    from edgeforge_amd import hip as H
    H.init(0)
    print(f"[gpu] {__import__('edgeforge_amd._lib', fromlist=['x']).device_name()}", flush=True)
    return H

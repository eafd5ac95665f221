import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library through its C ABI)")


@pytest.fixture(scope="session")
def hip():
    """The HIP backend on GPU 0. A GPU test fails loudly when the library or the GPU is missing."""
    from rustingstrata_amd import HipBackend
    b = HipBackend(0)
    print(f"[hip] {b.device()}", flush=True)
    yield b
    b.close()

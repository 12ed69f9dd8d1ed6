import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the mlx-hip C ABI)")


@pytest.fixture(scope="session")
def oracle_lib():
    from oracle import cpu_ref
    if not os.path.exists(cpu_ref.LIB):
        cpu_ref.build()
    return cpu_ref.load()


@pytest.fixture(scope="session")
def hip():
    """Initialised mlx-hip library (GPU tests only). Fails loudly when the
    library or the GPU is missing: there is no fallback."""
    from oxidizedmlx_amd import backend
    backend.init()
    return backend

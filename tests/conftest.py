import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run with -m gpu)")


@pytest.fixture(scope="session")
def rt():
    """One gfx950 runtime for the whole GPU session."""
    from eos_amd.runtime import Runtime
    r = Runtime(0)
    info = r.info()
    print(f"[gpu] runtime on {info}", flush=True)
    yield r
    r.close()

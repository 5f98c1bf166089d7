import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def hip():
    """The fakhip C ABI on device 0 (GPU tests only)."""
    from fak_amd import fakhip
    info = fakhip.init()
    print(f"[gpu] {info}", flush=True)
    return fakhip

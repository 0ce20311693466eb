import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")
    config.addinivalue_line("markers", "slow: long-running")


def pytest_runtest_logstart(nodeid, location):
    # With NT_TRACE_TESTS=1 every test announces itself before it runs, so a
    # run that dies inside a GPU call still names the test it was in.
    if os.environ.get("NT_TRACE_TESTS"):
        print(f"\nSTART {nodeid}", flush=True)


@pytest.fixture(scope="session")
def gpu():
    """Fails (not skips) when the device path is unusable: GPU tests must run
    the HIP library, never silently pass without it."""
    import nanotorch_amd as nt
    from nanotorch_amd import _lib

    _lib.load()  # raises ImportError if libnt.so is missing
    assert nt.is_available(), "no HIP device visible"
    return nt

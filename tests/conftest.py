"""Shared test configuration.

Tests marked ``gpu`` need an MI355X (gfx950) and call libkvx_amd.so through
its C ABI; everything else runs on the CPU.  The CPU oracle (oracle/) is the
checker in both.
"""
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (run with -m gpu)")


@pytest.fixture(scope="session")
def kvx_lib():
    from kvx_amd import abi

    return abi.load()


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    return oracle.lib()

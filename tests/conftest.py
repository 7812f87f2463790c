"""Test configuration: the `gpu` marker and shared helpers.

GPU tests drive librew_mi355x through its C ABI (via rew_amd.eager) and
compare against the CPU oracle in oracle/ on the same seeded inputs.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (run with -m gpu)")


@pytest.fixture(scope="session")
def oracle():
    import oracle as orc
    orc.build()
    return orc


@pytest.fixture(scope="session")
def gpu():
    """Installs the mi355x eager backend on device 0 (GPU tests only)."""
    from rew_amd import eager
    if eager.deviceCount() < 1:
        pytest.fail("no HIP device visible: GPU tests need an MI355X")
    eager.installEagerBackend(eager.mi355x(0))
    return eager

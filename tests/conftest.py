"""Shared test setup: markers, paths and the oracle / product library loaders."""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "aien-sovereign-core-mv_amd")
for p in (REPO, PKG, os.path.join(REPO, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(REPO, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running parity case")


@pytest.fixture(scope="session")
def oracle():
    import pyoracle

    return pyoracle


@pytest.fixture(scope="session")
def omega():
    """The product library (libomega_gpu.so) binding; GPU tests only."""
    import omega_amd

    omega_amd.require_gpu()
    return omega_amd

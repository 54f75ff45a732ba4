"""Shared test setup: import paths for the product binding and the oracle, the `gpu`
marker, and small model configurations used across the suites."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "ane-training-experiments_amd")
for p in (PKG, os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu():
    """Initialises device 0 through the C ABI (GPU tests only)."""
    import stories_hip as sh

    sh.init(0)
    return sh

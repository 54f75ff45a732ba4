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


def pytest_collection_modifyitems(session, config, items):
    """Runs the stories-generate child-process tests first. The persistent decode kernel is a
    cooperative launch, and the HIP runtime refuses one ("the operation cannot be performed
    in the present state") while another process that has made cooperative launches on the
    device is still alive, so the CLI children must finish before this process launches its
    own. The order is otherwise kept."""
    items.sort(key=lambda it: 0 if os.path.basename(str(it.fspath)) == "test_cli.py" else 1)

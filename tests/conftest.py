"""Shared test setup.

Markers: `gpu` tests need an MI355X (they call the HIP kernels through the C ABI);
everything else runs on the CPU. Without a GPU device (/dev/kfd) the gpu tests are
skipped; on a GPU machine they run and any failure is a failure.
"""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HAVE_GPU = os.path.exists("/dev/kfd")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    if HAVE_GPU:
        return
    skip = pytest.mark.skip(reason="no GPU in this container (/dev/kfd absent)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def rng():
    # the reference's test seed (tests/conftest.py:17-19)
    return np.random.default_rng(1234)

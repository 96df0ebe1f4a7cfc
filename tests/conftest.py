"""Shared pytest configuration.

Markers:
  gpu -- needs an MI355X (HIP device) and the built libarthip.so. Parity tests
         of the HIP path against the CPU oracle live behind this marker.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: requires a HIP GPU and the built libarthip.so")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def device() -> int:
    return int(os.environ.get("ARTHIP_TEST_DEVICE", "0"))


@pytest.fixture(scope="session")
def fixtures(tmp_path_factory):
    from tests.fixtures import FixtureSet
    return FixtureSet(tmp_path_factory.mktemp("fixtures"))


@pytest.fixture(scope="session")
def harness():
    from arthip_amd.engine import EngineHarness
    return EngineHarness()

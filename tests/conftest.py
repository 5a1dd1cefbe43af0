"""Shared fixtures.  `-m gpu` tests need a HIP device and the built library;
everything else runs on the CPU."""

from __future__ import annotations

import importlib
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")


def pkg(name: str = ""):
    """Import the package (its directory name starts with a digit)."""
    return importlib.import_module("15642_moe_amd" + (f".{name}" if name else ""))


@pytest.fixture(scope="session")
def moe():
    return pkg()


@pytest.fixture(scope="session")
def ops():
    return pkg("ops")


@pytest.fixture(scope="session")
def inputs_mod():
    return pkg("inputs")


@pytest.fixture(scope="session")
def capi():
    return pkg("capi")


@pytest.fixture(scope="session")
def lib(capi):
    return capi.load()


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a HIP device")
    return torch.device("cuda:0")

"""Shared pytest setup: the ``gpu`` marker, package loading, GPU gating."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

# Parity tests restate the library's built-in dispatch; a tuned table for the
# device (tuning.py) would change which kernels run.  Tests of the tables
# themselves clear this per test.
os.environ["W4A16_MOE_TUNING"] = "default"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def pkg():
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def synth(pkg):
    import importlib

    return importlib.import_module(__graft_entry__.PKG_NAME + ".synth")


@pytest.fixture(scope="session")
def lib(pkg):
    """The loaded C-ABI library (no GPU work)."""
    return pkg._lib.lib()


@pytest.fixture(scope="session")
def orc():
    from oracle import moe_oracle

    return moe_oracle


@pytest.fixture(scope="session")
def dev():
    import torch

    return torch.device("cuda:0")

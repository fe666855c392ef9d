"""Shared fixtures.  ``gpu`` tests need a ROCm device and the native library."""

from __future__ import annotations

import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libopake_amd.so")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def dev():
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before any GPU work so a failing run says which it was.
    if "gpu" in request.keywords:
        print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
    yield

"""Test configuration: import paths, the `gpu` marker, shared helpers.

CPU tests (-m "not gpu") pin the oracle and the host logic; GPU tests
(-m gpu) call the HIP library through the C ABI and compare with the oracle.
"""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "kv-cache-triton_amd")
for p in (ROOT, PKG, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libkvint4.so")


def _has_gpu() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _name_the_case(request):
    # Print the case before GPU work so a crash log names it.
    if "gpu" in request.keywords:
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield

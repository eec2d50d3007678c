"""Test configuration: the `gpu` marker, and the in-tree package on sys.path.

Tests marked `gpu` need an MI355X (gfx950) and the built libhkx.so; every other test
runs on the CPU (the oracle, the host logic, the library's exports)."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "hk-dsl_amd")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libhkx.so")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:  # noqa: BLE001
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU here")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)

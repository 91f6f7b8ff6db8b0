"""Shared pytest configuration: the ``gpu`` marker and GPU-availability gating."""

from __future__ import annotations

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); runs the gfx950 kernels")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_runtest_setup(item):
    # Name the case before it touches the GPU, so a fault that kills the process is attributable.
    if "gpu" in item.keywords:
        print(f"\n[gpu-case] {item.nodeid}", flush=True)

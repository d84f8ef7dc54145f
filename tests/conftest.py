"""Shared pytest configuration.

Tests marked ``gpu`` need an MI355X (HIP) device and the built
libaios_attn.so; everything else runs on the CPU.
"""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


def _gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


def pytest_collection_modifyitems(config, items):
    gpu_items = [it for it in items if "gpu" in it.keywords]
    if not gpu_items or _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible to torch")
    for it in gpu_items:
        it.add_marker(skip)

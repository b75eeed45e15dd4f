"""Shared pytest configuration.

Markers
-------
gpu : needs a ROCm GPU (MI355X); run with ``-m gpu``.  Everything else runs on
      the CPU (``-m "not gpu"``) and never launches a kernel.
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X)")


@pytest.fixture(scope="session")
def cuda_device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("ROCm GPU required")
    from reversability_amd import _hip
    _hip.library()  # fail loudly if the HIP library is not built
    return torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _announce(request):
    # Name each GPU test on stdout (flushed) before it runs, so a failing run
    # always shows which case was active.
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-test] {request.node.nodeid}", flush=True)
    yield

"""Shared pytest setup.

Markers: `gpu` marks tests that need the MI355X (run with -m gpu on the GPU
box); everything else runs on the CPU. The package lives in
llm-experiments_amd/, which is put on sys.path here.
"""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "llm-experiments_amd")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (ROOT, PKG, GOLDEN):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm MI355X GPU and libskv.so")


@pytest.fixture(scope="session")
def gpu_ctx():
    """GPUContext on cuda:0 for GPU tests; the HIP library must load."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from simple_llm_amd import _lib
    from simple_llm_amd.gpu import gpu

    _lib.lib()  # raises if libskv.so is missing: no silent fallback
    dev = gpu.device_create()
    return gpu.context_create(dev)


def banner(msg: str) -> None:
    """Name the case before GPU work so a fault report says which case ran."""
    print(f"[case] {msg}", flush=True)

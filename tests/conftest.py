"""pytest configuration: the ``gpu`` marker and the repository root on ``sys.path``.

Tests marked ``gpu`` need an MI355X (or any gfx950 device) and the built ``libgdn.so``; they are
skipped where ``torch.cuda.is_available()`` is False. On a GPU box a missing library is an error,
never a skip: the parity tests must exercise the HIP path.
"""
import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built libgdn.so")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this process (torch.cuda.is_available() is False)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session", autouse=True)
def _blas_workspace_first():
    """torch sets up its BLAS-Lt handle and workspace at the first GEMM of the process. One bf16
    linear (the layers' GEMM path) before any test allocates and frees device memory gives a full
    run the same GEMM setup as a run of a single test file."""
    if torch.cuda.is_available():
        x = torch.zeros(2, 64, 256, device="cuda", dtype=torch.bfloat16)
        w = torch.zeros(512, 256, device="cuda", dtype=torch.bfloat16)
        torch.nn.functional.linear(x, w)
        torch.cuda.synchronize()
    yield

"""Shared pytest setup: import paths, the `gpu` marker and GPU fixtures."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
for p in (REPO / "ai-compiler-framework_amd" / "python", REPO / "oracle", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def C():
    """The native binding module; GPU tests fail loudly if it is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from aicf_cuda import _C

    return _C


@pytest.fixture(scope="session")
def dev():
    import torch

    return torch.device("cuda:0")

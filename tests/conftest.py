"""Shared test configuration.

* ``gpu`` marks tests that need a visible GPU (run with ``-m gpu``).
* The package lives under ``micro-vllm_amd/`` (not importable by that name),
  so its parent directory is put on ``sys.path``; the repository root is on
  it too, for the oracle.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT, ROOT / "micro-vllm_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a visible MI355X (HIP) device")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture
def device():
    """cuda:0. After the test, dead objects are collected while no graph
    capture is under way: a HIP graph that a reference cycle keeps alive
    must not be destroyed inside a later test's capture."""

    import gc

    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    yield torch.device("cuda", 0)
    gc.collect()

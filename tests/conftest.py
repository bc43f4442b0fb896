"""Shared test setup: import paths, the ``gpu`` marker and device helpers.

``-m "not gpu"`` covers the oracle (against golden vectors, the float64 mathematics and the
reference's compiled kernels when built), host-side logic and the C ABI's symbols and
argument checks. ``-m gpu`` runs the HIP kernels through the C ABI and the torch ops and
compares them with the oracle.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
for p in (REPO, REPO / "llm-serving-engine_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP libraries")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; loads the native libraries (fails loudly if they are missing)."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no ROCm device is visible")
    from llmserve._native import capi, ops

    ops()
    capi()
    return torch.device("cuda", 0)

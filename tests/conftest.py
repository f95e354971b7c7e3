"""Test tiers (the reference's split: CPU-checkable logic everywhere, kernels on the GPU):

- `-m "not gpu"`: the numpy oracle against known answers, invariants, brute force and torch's own
  library routines; the committed golden fixtures; the C-ABI library's exports and its
  host-side argument validation (no kernel launches); host logic of the Python wrappers.
- `-m gpu`: every HIP kernel against the oracle on the same seeded inputs, through the C ABI.

GPU tests are skipped automatically when no GPU is visible.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG = REPO / "llm-decode-kernels_amd"
for p in (str(REPO), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)

import torch  # noqa: E402

ON_GPU = torch.cuda.is_available()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); skipped without one")
    config.addinivalue_line("markers", "slow: full-size shapes")


def pytest_collection_modifyitems(config, items):
    skip_gpu = pytest.mark.skip(reason="needs a ROCm GPU")
    for item in items:
        if "gpu" in item.keywords and not ON_GPU:
            item.add_marker(skip_gpu)


def _ensure_built():
    lib = PKG / "kernels" / "libldk_amd.so"
    if not lib.exists():
        sys.path.insert(0, str(PKG))
        import build as _build  # llm-decode-kernels_amd/build.py

        _build.build()


_ensure_built()


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(0)

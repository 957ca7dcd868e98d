"""Shared test setup: import paths, the ``gpu`` marker, seeded inputs."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "topk-tarmac_amd", ROOT / "oracle", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = ROOT / "tests" / "golden" / "reference_vectors.npz"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")


def pytest_collection_modifyitems(config, items):
    # Run GPU tests only when a HIP device exists; on CPU they are skipped
    # (the CPU suite runs them deselected with -m "not gpu").
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def qkv(seed: int, B: int, N: int, d: int, dtype=np.float32):
    """Q, K, V ~ N(0, 1) i.i.d. from a CPU generator (identical bits for the
    oracle and the kernel)."""
    rng = np.random.default_rng(seed)
    return [rng.standard_normal((B, N, d)).astype(dtype) for _ in range(3)]


@pytest.fixture(scope="session")
def golden():
    return np.load(GOLDEN)

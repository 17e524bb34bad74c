"""Shared test setup: import paths, the `gpu` marker and seeded data helpers."""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
for path in (REPO / "m5-max-kernels_amd", REPO):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device) and the built libm5k.so")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # pragma: no cover - torch import failure
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def kats():
    return json.loads((GOLDEN / "reference_kats.json").read_text())


@pytest.fixture(scope="session")
def device():
    import torch

    from m5kernels_amd import _lib

    _lib.load()  # fail loudly if the HIP library was not built
    return torch.device("cuda:0")


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """numpy float32 -> bf16 bits by round to nearest even (torch's .to(bfloat16))."""
    from oracle.reference import f32_to_bf16_bits

    return f32_to_bf16_bits(x)

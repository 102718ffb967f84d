"""Test configuration: markers, import paths and shared fixtures.

``-m "not gpu"`` runs the oracle pins, the host logic and the C-ABI export
checks on the CPU; ``-m gpu`` runs the HIP kernels against the oracle on a
real MI355X (those tests fail, never skip, when no GPU is visible).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "montlok.cpp_amd", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device) and the built libmlk_hip.so")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def golden():
    cache = {}

    def load(name: str):
        if name not in cache:
            with np.load(ROOT / "tests" / "golden" / f"{name}.npz", allow_pickle=False) as z:
                cache[name] = {k: z[k] for k in z.files}
        return cache[name]

    return load


@pytest.fixture(scope="session")
def dev():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible ROCm device"
    from montlok.rdt._loader import load_montlok

    load_montlok()  # raises if libmlk_hip.so is missing: no silent fallback
    return torch.device("cuda:0")

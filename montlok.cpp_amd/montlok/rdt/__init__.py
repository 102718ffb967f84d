"""RDT4quant fused forward on MI355X: the montlok.rdt drop-in path on ROCm.

Importing this package enables the GPU kernels unless ``MONTLOK_CPP`` is
already set (the reference does the same for its CPU kernels,
python/montlok/rdt/__init__.py:27); ``MONTLOK_CPP=0`` keeps the pure PyTorch
path of each module.
"""

from __future__ import annotations

import importlib
import os
from typing import Any

os.environ.setdefault("MONTLOK_CPP", "1")

_EXPORTS = {
    "Mamba3CPUReference": "mamba3",
    "Mamba3HIP": "mamba3",
    "ManifoldHyperConnectionCPU": "mhc",
    "ManifoldHyperConnectionHIP": "mhc",
    "MLACPU": "mla",
    "MLAHIP": "mla",
    "RMSNormCPU": "layers",
    "GroupedRMSNormCPU": "layers",
    "LayerNormCPU": "layers",
    "SwiGLUCPU": "layers",
    "RMSNormHIP": "layers",
    "GroupedRMSNormHIP": "layers",
    "LayerNormHIP": "layers",
    "SwiGLUHIP": "layers",
    "install_cpu_layers": "layers",
    "RDT4QuantCPU": "model",
    "RDT4QuantHIP": "model",
    "MultiAssetRDTCPU": "model",
    "MultiAssetRDTHIP": "model",
    "RDTModelConfig": "model",
    "cpu_linear": "linear",
}

__all__ = ["build_info", *_EXPORTS]


def build_info() -> dict:
    """Kernel variant and device of libmlk_hip.so."""
    from ._loader import load_montlok

    return dict(load_montlok().build_info())


def __getattr__(name: str) -> Any:
    if name in _EXPORTS:
        return getattr(importlib.import_module(f".{_EXPORTS[name]}", __name__), name)
    raise AttributeError(f"module 'montlok.rdt' has no attribute {name!r}")

"""RDT4quant fused forward on MI355X: the montlok.rdt drop-in path on ROCm.

Importing this package enables the GPU kernels unless ``MONTLOK_CPP`` is
already set (the reference does the same for its CPU kernels,
python/montlok/rdt/__init__.py:27).

Switches (README.md:265-280 of the reference), read on every call:

- ``MONTLOK_CPP=0``, ``MONTLOK_CPP_MHC=0``, ``MONTLOK_CPP_LAYERS=0``: the
  affected modules run the upstream PyTorch forward (``torch_path``) on the
  input's device instead of their kernels, as the reference does; with the
  switches on, a module that cannot take its kernels raises.
- ``MONTLOK_CPP_FUSED=0``: Mamba-3 pre-processing as tensor operations, then
  the recurrence kernel alone (``mamba3.cpp_backend``).
- ``MONTLOK_CPP_TAIL=0``: the model evaluates every position and takes the
  last one instead of the last-position tail (``model.tail_enabled``).
- ``MONTLOK_CPP_NATIVE_STAGE1=0`` / ``MONTLOK_CPP_NATIVE_STAGE2=0``: the
  stage-1 / stage-2 modules run one by one instead of the one-call
  ``stage1_forward`` / ``stage2_tail_forward``.
- ``MONTLOK_CACHE_PARAMETER_PACKS=0``: parameter packs are rebuilt per call.
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
    "Mamba3BlockHIP": "block",
    "DecodeStackHIP": "block",
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

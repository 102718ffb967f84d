"""When the drop-in modules may run their GPU kernels.

The reference enables its CPU kernels with ``MONTLOK_CPP=1`` and per-family
switches (``MONTLOK_CPP_LAYERS``, ``MONTLOK_CPP_MHC``; python/montlok/rdt/
layers.py:32-39, mhc.py:62-69, mla.py:86-104) and runs the upstream PyTorch
modules where a switch turns them off. The modules here do the same for the
switches (``backend_enabled`` false: the tensor programs of ``torch_path``).
With the switches on, a module takes its GPU kernels or raises: the conditions
below are checked, and there is no silent second path.
"""

from __future__ import annotations

import os

import torch


def backend_enabled(family: str | None = None) -> bool:
    if os.environ.get("MONTLOK_CPP") != "1":
        return False
    return family is None or os.environ.get(family) != "0"


def require_gpu_inference(module: str, x: torch.Tensor, family: str | None = None) -> None:
    """Raise unless ``x`` can take the GPU path: kernels enabled, fp32 on the ROCm device, no autograd."""
    if not backend_enabled(family):
        switch = f"MONTLOK_CPP=1{'' if family is None else f' and {family}!=0'}"
        raise RuntimeError(f"{module}: the GPU kernels are switched off ({switch} enables them); this package has "
                           f"no other forward")
    if x.device.type != "cuda":
        raise RuntimeError(f"{module}: input must be on the ROCm device, got {x.device}")
    if x.dtype != torch.float32:
        raise RuntimeError(f"{module}: input must be float32, got {x.dtype}")
    if torch.is_grad_enabled():
        raise RuntimeError(f"{module}: inference only; call it under torch.no_grad() or torch.inference_mode()")


def ext():
    from ._loader import load_montlok

    return load_montlok()

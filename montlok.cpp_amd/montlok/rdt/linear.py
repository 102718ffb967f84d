"""Inference linear on the matrix cores (reference: python/montlok/rdt/linear.py:11-32).

``cpu_linear`` keeps the reference's name so callers import it unchanged; it
runs ``montlok._C.linear`` (fp32 or bf16 weights, fp32 accumulation). With
``MONTLOK_CPP=0`` it is ``torch.nn.functional.linear``, as the reference's
fallback is (linear.py:24-32).
"""

from __future__ import annotations

import torch
from torch.nn import functional as F

from ._gate import backend_enabled, ext


def native_linear_enabled(x: torch.Tensor, weight: torch.Tensor) -> bool:
    return (backend_enabled() and x.device.type == "cuda" and weight.device.type == "cuda"
            and x.dtype == torch.float32 and weight.dtype in (torch.float32, torch.bfloat16)
            and not torch.is_grad_enabled())


def cpu_linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """``x @ weight.T + bias`` through the GPU linear; raises when the GPU path is not available."""
    if not backend_enabled():
        return F.linear(x, weight.to(x.dtype), None if bias is None else bias.to(x.dtype))
    if not native_linear_enabled(x, weight):
        raise RuntimeError("cpu_linear: needs MONTLOK_CPP=1, float32 input and float32/bfloat16 weight on the ROCm "
                           "device, and no autograd")
    return ext().linear(x, weight, bias)

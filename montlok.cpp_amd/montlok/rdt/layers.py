"""Per-token layers on the GPU: RMSNorm / GroupedRMSNorm, LayerNorm, SwiGLU.

Same constructor arguments, attributes and parameters as the upstream modules
the reference subclasses (reference/Model/layers/rmsnorm.py:9-60,
swiglu.py:10-35, torch.nn.LayerNorm), so state dicts load unchanged; each
forward is one GPU op from ``montlok._C`` (python/montlok/rdt/layers.py:48-92).
``install_cpu_layers(model)`` re-classes matching instances of a built model
(layers.py:95-115). ``MONTLOK_CPP_LAYERS=0`` (or ``MONTLOK_CPP=0``) runs the
upstream PyTorch forward instead (``torch_path``), as the reference does.
"""

from __future__ import annotations

import torch
from torch import nn

from . import torch_path
from ._gate import backend_enabled, ext, require_gpu_inference

_FAMILY = "MONTLOK_CPP_LAYERS"


class RMSNormHIP(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-5) -> None:
        super().__init__()
        if dim <= 0:
            raise ValueError("dim must be positive")
        if eps <= 0:
            raise ValueError("eps must be positive")
        self.dim = dim
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.dim:
            raise ValueError(f"expected last dim {self.dim}, got {x.shape[-1]}")
        if not backend_enabled(_FAMILY):
            return torch_path.rms_norm(x, self.weight, self.eps)
        require_gpu_inference(type(self).__name__, x, _FAMILY)
        return ext().rms_norm(x, self.weight, self.eps, 1)


class GroupedRMSNormHIP(nn.Module):
    def __init__(self, dim: int, num_groups: int = 1, eps: float = 1e-5) -> None:
        super().__init__()
        if dim <= 0:
            raise ValueError("dim must be positive")
        if num_groups <= 0:
            raise ValueError("num_groups must be positive")
        if dim % num_groups != 0:
            raise ValueError("dim must be divisible by num_groups")
        if eps <= 0:
            raise ValueError("eps must be positive")
        self.dim = dim
        self.num_groups = num_groups
        self.group_size = dim // num_groups
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.dim:
            raise ValueError(f"expected last dim {self.dim}, got {x.shape[-1]}")
        if not backend_enabled(_FAMILY):
            return torch_path.rms_norm(x, self.weight, self.eps, self.num_groups)
        require_gpu_inference(type(self).__name__, x, _FAMILY)
        return ext().rms_norm(x, self.weight, self.eps, self.num_groups)


class LayerNormHIP(nn.LayerNorm):
    """``torch.nn.LayerNorm`` over one trailing dimension, biased variance, fp64 statistics."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if len(self.normalized_shape) != 1 or self.weight is None:
            raise RuntimeError("LayerNormHIP: needs one normalized dimension and an affine weight")
        if x.shape[-1] != self.normalized_shape[0]:
            raise ValueError(f"expected last dim {self.normalized_shape[0]}, got {x.shape[-1]}")
        if not backend_enabled(_FAMILY):
            return super().forward(x)
        require_gpu_inference(type(self).__name__, x, _FAMILY)
        return ext().layer_norm(x, self.weight, self.bias, self.eps)


class SwiGLUHIP(nn.Module):
    """``w_down(silu(gate) * up)`` with ``[gate | up] = w_in(x)``: linear, fused gate, linear."""

    def __init__(self, d_model: int, ffn_hidden: int, bias: bool = False):
        super().__init__()
        if d_model <= 0:
            raise ValueError("d_model must be positive")
        if ffn_hidden <= 0:
            raise ValueError("ffn_hidden must be positive")
        self.d_model = d_model
        self.ffn_hidden = ffn_hidden
        self.w_in = nn.Linear(d_model, 2 * ffn_hidden, bias=bias)
        self.w_down = nn.Linear(ffn_hidden, d_model, bias=bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.d_model:
            raise ValueError(f"expected last dim {self.d_model}, got {x.shape[-1]}")
        if not backend_enabled(_FAMILY):
            return torch_path.swiglu(x, self.w_in, self.w_down)
        require_gpu_inference(type(self).__name__, x, _FAMILY)
        return ext().swiglu_mlp(x, self.w_in.weight, self.w_in.bias, self.w_down.weight, self.w_down.bias)


# The reference's class names, for code that imports them.
RMSNormCPU = RMSNormHIP
GroupedRMSNormCPU = GroupedRMSNormHIP
LayerNormCPU = LayerNormHIP
SwiGLUCPU = SwiGLUHIP

_SWAPS_BY_NAME = {"RMSNorm": RMSNormHIP, "GroupedRMSNorm": GroupedRMSNormHIP, "SwiGLU": SwiGLUHIP,
                  "LayerNorm": LayerNormHIP}


def install_cpu_layers(module: nn.Module) -> int:
    """Re-class every RMSNorm / GroupedRMSNorm / LayerNorm / SwiGLU instance under ``module``.

    Matches the upstream classes by name (and torch.nn.LayerNorm by type); the
    attributes and parameters are the same, so nothing is copied. Returns the
    number of instances swapped."""
    swapped = 0
    for child in module.modules():
        cls = type(child)
        replacement = _SWAPS_BY_NAME.get(cls.__name__)
        if cls is nn.LayerNorm:
            replacement = LayerNormHIP
        if replacement is not None and cls is not replacement:
            child.__class__ = replacement
            swapped += 1
    return swapped

"""Mamba-3 SISO mixer on the GPU with the reference's parameter contract.

``Mamba3HIP`` (also importable as ``Mamba3CPUReference``) has the constructor,
attributes and state-dict names of the reference module
(python/montlok/rdt/mamba3.py:83-141): ``in_proj.weight [W, d_model]``,
``dt_bias [H]``, ``B_bias``/``C_bias [H, 1, N]``, ``B_norm.weight``/
``C_norm.weight [N]``, ``D [H]``, ``out_proj.weight``, with
W = 2 d_inner + 2 N ngroups + 3 H + R and R = (floor(N rope_fraction) rounded
down to even) / 2 rotary angles. ``forward`` is the fused layer
(mamba3_siso_layer: in_proj, the Mamba-3 mixer, out_proj; mamba3.py:143-173).

``new_state`` / ``step`` run one token for many independent streams with
carried state (S, k_prev, v_prev and the fp64 rotary phase). No reference
operator exists for this; stepping T tokens from ``new_state`` gives the
forward over those T tokens.
"""

from __future__ import annotations

import math

import torch
from torch import nn

from ._gate import backend_enabled, ext, require_gpu_inference


def cpp_backend() -> str | None:
    """``"fused"`` when the GPU kernels are enabled (``MONTLOK_CPP=1``), else ``None`` (mamba3.py:50-54)."""
    return "fused" if backend_enabled() else None


class BCNorm(nn.Module):
    """Holds the B / C RMS-norm weight and eps (mamba3.py:37-47); the kernels apply it."""

    def __init__(self, dimension: int, eps: float = 1e-5, **_: object):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dimension))
        self.eps = eps


class Mamba3HIP(nn.Module):
    def __init__(self, d_model: int, d_state: int = 128, expand: int = 2, headdim: int = 64, ngroups: int = 1,
                 rope_fraction: float = 0.5, dt_min: float = 0.001, dt_max: float = 0.1,
                 dt_init_floor: float = 1e-4, A_floor: float = 1e-4, is_outproj_norm: bool = False,
                 is_mimo: bool = False, mimo_rank: int = 4, layer_idx: int | None = None, device=None, dtype=None,
                 **_: object):
        super().__init__()
        if is_mimo or is_outproj_norm:
            raise ValueError("the GPU mixer supports the SISO / no-outproj-norm contract only")
        self.d_model = d_model
        self.d_state = d_state
        self.expand = expand
        self.headdim = headdim
        self.d_inner = d_model * expand
        if self.d_inner % headdim:
            raise ValueError("d_model * expand must be divisible by headdim")
        self.nheads = self.d_inner // headdim
        self.num_bc_heads = ngroups
        self.mimo_rank = 1
        self.layer_idx = layer_idx
        self.A_floor = A_floor
        split = int(d_state * rope_fraction)
        if split % 2:
            split -= 1
        self.num_rope_angles = split // 2
        factory = {"device": device, "dtype": dtype}
        width = 2 * self.d_inner + 2 * d_state * ngroups + 3 * self.nheads + self.num_rope_angles
        self.in_proj = nn.Linear(d_model, width, bias=False, **factory)
        log_low, log_high = math.log(dt_min), math.log(dt_max)
        dt = torch.exp(torch.rand(self.nheads, device=device) * (log_high - log_low) + log_low).clamp_min(dt_init_floor)
        self.dt_bias = nn.Parameter(dt + torch.log(-torch.expm1(-dt)))
        self.B_bias = nn.Parameter(torch.ones(self.nheads, 1, d_state, device=device))
        self.C_bias = nn.Parameter(torch.ones(self.nheads, 1, d_state, device=device))
        self.B_norm = BCNorm(d_state, eps=1e-5)
        self.C_norm = BCNorm(d_state, eps=1e-5)
        self.D = nn.Parameter(torch.ones(self.nheads, device=device))
        self.out_proj = nn.Linear(self.d_inner, d_model, bias=False, **factory)

    def _mixer_args(self) -> tuple:
        return (self.B_bias, self.C_bias, self.B_norm.weight, self.C_norm.weight, self.dt_bias, self.D)

    def _geometry(self) -> tuple:
        return (self.d_state, self.num_bc_heads, self.nheads, self.headdim, self.num_rope_angles, self.B_norm.eps,
                self.C_norm.eps, self.A_floor)

    def forward(self, inputs: torch.Tensor, **_: object) -> torch.Tensor:
        if inputs.ndim != 3 or inputs.shape[-1] != self.d_model:
            raise ValueError("Mamba3HIP expects [batch, length, d_model]")
        require_gpu_inference(type(self).__name__, inputs)
        return ext().mamba3_siso_layer(inputs, self.in_proj.weight, self.out_proj.weight, *self._mixer_args(),
                                       *self._geometry())

    def forward_projected(self, projected: torch.Tensor) -> torch.Tensor:
        """in_proj output [B, L, W] -> out_proj input [B, L, d_inner] (mamba3.py:175-197)."""
        require_gpu_inference(type(self).__name__, projected)
        return ext().mamba3_siso_forward(projected, None, *self._mixer_args(), *self._geometry())

    def new_state(self, streams: int, device=None) -> dict:
        """Zero carried state for ``streams`` independent sequences."""
        device = device if device is not None else self.D.device
        return ext().new_mamba3_state(streams, self.nheads, self.d_state, self.headdim, self.num_rope_angles, device)

    def step(self, u: torch.Tensor, state: dict) -> torch.Tensor:
        """One token ``u [S, d_model]`` per stream; updates ``state`` in place; returns ``[S, d_model]``."""
        if u.ndim != 2 or u.shape[-1] != self.d_model:
            raise ValueError("Mamba3HIP.step expects [streams, d_model]")
        require_gpu_inference(type(self).__name__, u)
        c = ext()
        projected = c.linear(u, self.in_proj.weight)
        y = c.mamba3_siso_step(projected, state, *self._mixer_args(), *self._geometry())
        return c.linear(y, self.out_proj.weight)


Mamba3CPUReference = Mamba3HIP

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

Backends (chosen per call from the environment, as mamba3.py:50-54 does):

``MONTLOK_CPP=1`` (the default once ``montlok.rdt`` is imported)
    the fused layer: in_proj, one kernel from the in_proj rows to the gated
    output (BCNorm, biases, dt/A/trap, rotary phase, recurrence, silu gate),
    out_proj.
``MONTLOK_CPP=1 MONTLOK_CPP_FUSED=0``
    the reference's debug ladder for isolating a mismatch between the fused
    pre-processing and the recurrence (mamba3.py:14-16, 226-240): the
    pre-processing as tensor operations on the device, then only the
    recurrence kernel (``mamba3_siso_recurrent``). Its fp32 rotary cumsum
    and libm-free tensor math differ from the fused kernel's fp64 running
    phase by rounding; the reference's own gate for this pair is
    2e-5 (1 + max|y|) (tests/rdt/test_rdt_kernels.py:126-128).
``MONTLOK_CPP`` other than ``1``
    the pure PyTorch quadratic form of the reference's own fallback
    (mamba3.py:199-256; ``torch_path.mamba3_forward``) on the input's device.
"""

from __future__ import annotations

import math
import os

import torch
from torch import nn
from torch.nn import functional as F

from . import torch_path
from ._gate import backend_enabled, ext, require_gpu_inference


def cpp_backend() -> str | None:
    """``"fused"`` or ``"recurrent"`` (``MONTLOK_CPP_FUSED=0``) when the GPU kernels are enabled
    (``MONTLOK_CPP=1``), else ``None`` (mamba3.py:50-54)."""
    if not backend_enabled():
        return None
    return "recurrent" if os.environ.get("MONTLOK_CPP_FUSED") == "0" else "fused"


def heavy_tail_activation(value: torch.Tensor) -> torch.Tensor:
    """x for x >= 0, 1 / (1 - x) below (mamba3.py:30-33)."""
    return value.clamp_min(0) + torch.reciprocal(1 - value.clamp_max(0))


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
        if cpp_backend() is None:
            return torch_path.mamba3_forward(self, inputs)
        require_gpu_inference(type(self).__name__, inputs)
        c = ext()
        if cpp_backend() == "recurrent":
            projected = c.linear(inputs, self.in_proj.weight)
            return c.linear(self._forward_recurrent(projected), self.out_proj.weight)
        return c.mamba3_siso_layer(inputs, self.in_proj.weight, self.out_proj.weight, *self._mixer_args(),
                                   *self._geometry())

    def _forward_recurrent(self, projected: torch.Tensor) -> torch.Tensor:
        """``MONTLOK_CPP_FUSED=0``: the pre-processing as tensor operations, then the recurrence kernel.

        Splits the in_proj row [z | x | B | C | dt | A | trap | angles], BCNorm's B and C per group plus the
        per-head biases (group h // (H / G)), dt = softplus(dt + dt_bias), adt = -max(heavy_tail(A), A_floor)
        * dt, the rotary phase cumsum(tanh(angles) * pi * dt) wrapped to [0, 2 pi), and the rotation of the
        interleaved pairs (2r, 2r + 1) of q and k for r < R (mamba3.py:199-240). Returns [B, L, d_inner]."""
        B, L, _ = projected.shape
        H, N, G, D, R = self.nheads, self.d_state, self.num_bc_heads, self.headdim, self.num_rope_angles
        z, x, b_val, c_val, raw_dt, raw_a, raw_trap, raw_ang = torch.split(
            projected, [self.d_inner, self.d_inner, N * G, N * G, H, H, H, R], dim=-1)

        def bc(value, norm, bias):
            v = value.reshape(B, L, G, N)
            v = v * torch.rsqrt(v.square().mean(dim=-1, keepdim=True) + norm.eps) * norm.weight
            return (v.unsqueeze(3) + bias.view(1, 1, G, H // G, N)).reshape(B, L, H, N)

        k = bc(b_val, self.B_norm, self.B_bias)
        q = bc(c_val, self.C_norm, self.C_bias)
        dt = F.softplus(raw_dt + self.dt_bias)
        adt = -heavy_tail_activation(raw_a).clamp_min(self.A_floor) * dt
        if R > 0:
            phase = torch.cumsum(torch.tanh(raw_ang).unsqueeze(2) * math.pi * dt.unsqueeze(-1), dim=1)
            phase = phase - 2 * math.pi * torch.floor(phase / (2 * math.pi))
            cos, sin = torch.cos(phase), torch.sin(phase)

            def rotate(v):
                pairs = v[..., :2 * R].unflatten(-1, (R, 2))
                left, right = pairs[..., 0], pairs[..., 1]
                turned = torch.stack((left * cos - right * sin, left * sin + right * cos), dim=-1).flatten(-2)
                return torch.cat((turned, v[..., 2 * R:]), dim=-1)

            q, k = rotate(q), rotate(k)
        gate = F.silu(z).reshape(B, L, H, D)
        y = ext().mamba3_siso_recurrent(q.contiguous(), k.contiguous(), x.unflatten(-1, (H, D)), gate, adt, dt,
                                        raw_trap, self.D)
        return y.reshape(B, L, self.d_inner)

    def forward_projected(self, projected: torch.Tensor) -> torch.Tensor:
        """in_proj output [B, L, W] -> out_proj input [B, L, d_inner] (mamba3.py:175-197)."""
        if cpp_backend() is None:
            return torch_path.mamba3_mixer(self, projected)
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

"""The RMSNorm -> Mamba-3 residual block and a stack of them for streaming decode.

``Mamba3BlockHIP`` is the upstream ``Mamba3Layer`` on the official backend
(python/montlok/rdt/reference/Model/layers/mamba3_layer.py:387-398, forward
:488-498): ``x + mixer(GroupedRMSNorm(x))`` with the mixer's parameter contract
(``norm.weight``, ``mamba.*`` as ``Mamba3HIP``). ``forward`` over a window of
tokens is one ``montlok._C.mamba3_block`` call; ``step`` advances S independent
streams by one token with carried state (the upstream step API,
mamba3_layer.py:567-580; the reference has no step operator).

``DecodeStackHIP`` chains such blocks and ends in RMSNorm and a linear head:
per stream and bar, ``head(RMSNorm(block_n(... block_1(x))))``. Stepping T bars
from ``new_state`` gives the forward over those T bars, row for row.
"""

from __future__ import annotations

import torch
from torch import nn

from ._gate import backend_enabled, ext, require_gpu_inference
from .linear import cpu_linear
from .layers import GroupedRMSNormHIP, RMSNormHIP
from .mamba3 import Mamba3HIP


class Mamba3BlockHIP(nn.Module):
    def __init__(self, d_model: int, d_state: int = 128, expand: int = 2, headdim: int = 64, num_groups: int = 8,
                 eps: float = 1e-5, **mixer_kwargs):
        super().__init__()
        self.norm = GroupedRMSNormHIP(d_model, num_groups=num_groups, eps=eps)
        self.mamba = Mamba3HIP(d_model, d_state=d_state, expand=expand, headdim=headdim, **mixer_kwargs)

    def _args(self) -> tuple:
        m = self.mamba
        return (self.norm.weight, self.norm.eps, self.norm.num_groups, m.in_proj.weight, m.out_proj.weight,
                *m._mixer_args(), *m._geometry())

    def forward(self, x: torch.Tensor, **_: object) -> torch.Tensor:
        if x.ndim != 3 or x.shape[-1] != self.mamba.d_model:
            raise ValueError("Mamba3BlockHIP expects [batch, length, d_model]")
        if not backend_enabled():
            return x + self.mamba(self.norm(x))  # each module's upstream PyTorch forward
        require_gpu_inference(type(self).__name__, x)
        return ext().mamba3_block(x, *self._args())

    def new_state(self, streams: int, device=None) -> dict:
        return self.mamba.new_state(streams, device)

    def step(self, u: torch.Tensor, state: dict) -> torch.Tensor:
        """One token ``u [S, d_model]`` per stream; ``state`` is updated in place."""
        if u.ndim != 2 or u.shape[-1] != self.mamba.d_model:
            raise ValueError("Mamba3BlockHIP.step expects [streams, d_model]")
        require_gpu_inference(type(self).__name__, u)
        return ext().mamba3_block_step(u, state, *self._args())


class DecodeStackHIP(nn.Module):
    """``n_layers`` Mamba-3 blocks, then RMSNorm and a ``Linear(d_model -> n_outputs)`` head."""

    def __init__(self, d_model: int = 128, n_layers: int = 2, d_state: int = 64, expand: int = 2, headdim: int = 64,
                 num_groups: int = 8, n_outputs: int = 1, eps: float = 1e-5):
        super().__init__()
        self.d_model = d_model
        self.layers = nn.ModuleList(Mamba3BlockHIP(d_model, d_state, expand, headdim, num_groups, eps)
                                    for _ in range(n_layers))
        self.final_norm = RMSNormHIP(d_model, eps=eps)
        self.head = nn.Linear(d_model, n_outputs)

    def new_state(self, streams: int, device=None) -> list[dict]:
        return [layer.new_state(streams, device) for layer in self.layers]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Every bar of ``x [B, L, d_model]`` -> ``[B, L, n_outputs]``."""
        for layer in self.layers:
            x = layer(x)
        return cpu_linear(self.final_norm(x), self.head.weight, self.head.bias)

    def step(self, x: torch.Tensor, states: list[dict]) -> torch.Tensor:
        """One bar ``x [S, d_model]`` per stream -> ``[S, n_outputs]``; ``states`` advance in place."""
        if len(states) != len(self.layers):
            raise ValueError(f"expected {len(self.layers)} layer states, got {len(states)}")
        for layer, state in zip(self.layers, states):
            x = layer.step(x, state)
        return ext().linear(self.final_norm(x), self.head.weight, self.head.bias)

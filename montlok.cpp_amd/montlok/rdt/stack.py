"""A hybrid stack of mHC residual layers built from the drop-in modules.

Features ``[B, L, d_features]`` go through a linear projection to ``d_model``
and are expanded to ``n`` streams. They then pass ``n_layers`` mHC residuals
whose wrapped layers alternate ``Mamba3(RMSNorm(agg))`` and
``MLA(RMSNorm(agg))`` (the residual-with-norm form of
reference/Model/two_stage.py:100-116), and are collapsed to the mean of the
streams (two_stage.py:405-409).

The forward chains the fused operators the way the reference's native
stage-2 path does. The first residual is prepared straight from the broadcast
backbone (no expanded copy). Each residual's write is fused with the next
residual's prepare (``mhc_combine_prepare``). Each layer's input RMSNorm is
applied to the aggregate inside the prepare (``agg_norm_w``). The last
residual writes the collapsed mean directly.
"""

from __future__ import annotations

from types import SimpleNamespace

import torch
from torch import nn
from torch.nn import functional as F

from ._gate import backend_enabled, ext, require_gpu_inference
from .layers import RMSNormHIP
from .mamba3 import Mamba3HIP
from .mhc import ManifoldHyperConnectionHIP
from .mla import MLAHIP


class HybridStackHIP(nn.Module):
    def __init__(self, d_features: int, d_model: int = 256, n_layers: int = 4, n_streams: int = 4,
                 sinkhorn_iters: int = 20, rmsnorm_eps: float = 1e-5, d_state: int = 64, mamba_headdim: int = 64,
                 expand: int = 2, n_heads: int = 4, head_dim: int = 64, rope_head_dim: int = 32,
                 kv_lora_rank: int = 64, rope_theta: float = 10000.0):
        super().__init__()
        self.d_model = d_model
        self.n_streams = n_streams
        self.feature_proj = nn.Linear(d_features, d_model)
        mla_cfg = SimpleNamespace(d_model=d_model, n_heads=n_heads, head_dim=head_dim,
                                  nope_head_dim=head_dim - rope_head_dim, rope_head_dim=rope_head_dim,
                                  kv_lora_rank=kv_lora_rank, q_lora_rank=0, rope_theta=rope_theta, dropout=0.0)
        self.hcs = nn.ModuleList(ManifoldHyperConnectionHIP(d_model, n_streams, sinkhorn_iters, True, rmsnorm_eps)
                                 for _ in range(n_layers))
        self.norms = nn.ModuleList(RMSNormHIP(d_model, eps=rmsnorm_eps) for _ in range(n_layers))
        self.mixers = nn.ModuleList(
            Mamba3HIP(d_model, d_state=d_state, expand=expand, headdim=mamba_headdim) if i % 2 == 0 else MLAHIP(mla_cfg)
            for i in range(n_layers))

    def linear_weights(self) -> list[torch.Tensor]:
        """The GEMM weights (the ones a bf16-weight configuration stores in bf16)."""
        out = [self.feature_proj.weight]
        for m in self.mixers:
            out += [mod.weight for mod in m.modules() if isinstance(mod, nn.Linear)]
        return out

    def forward(self, features: torch.Tensor) -> torch.Tensor:
        if features.ndim != 3:
            raise ValueError("features must be [B, L, d_features]")
        if not backend_enabled():
            # The kernels switched off: the module chain, each module's upstream PyTorch forward.
            streams = self.hcs[0].expand(F.linear(features, self.feature_proj.weight.to(features.dtype),
                                                  self.feature_proj.bias.to(features.dtype)))
            for hc, norm, mixer in zip(self.hcs, self.norms, self.mixers):
                streams = hc(streams, lambda agg, norm=norm, mixer=mixer: mixer(norm(agg)))
            return self.hcs[-1].collapse(streams)
        require_gpu_inference(type(self).__name__, features)
        c = ext()
        h = c.linear(features, self.feature_proj.weight, self.feature_proj.bias)
        first, norm = self.hcs[0], self.norms[0]
        streams, prepared = first._prepare(h, allow_broadcast=True, output_norm=norm)
        out = self.mixers[0](prepared[0])
        for i in range(1, len(self.hcs)):
            streams, prepared = self.hcs[i - 1]._combine_prepare(streams, prepared, out, self.hcs[i],
                                                                 output_norm=self.norms[i])
            out = self.mixers[i](prepared[0])
        return self.hcs[-1]._combine_collapse(streams, prepared, out)

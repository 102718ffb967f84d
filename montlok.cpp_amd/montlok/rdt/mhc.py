"""Manifold-constrained hyper-connection (mHC) on the GPU.

``ManifoldHyperConnectionHIP`` (also importable as
``ManifoldHyperConnectionCPU``) has the constructor, initial values and
state-dict names of the upstream module (reference/Model/layers/mhc.py:72-165):
``pre_bias [n]``, ``post_bias [n]``, ``res_bias [n, n]``, ``dyn_norm.weight
[d]``, ``pre_proj``/``post_proj``/``res_proj.weight``, and the 0-d
``pre_alpha``/``post_alpha``/``res_alpha``. ``forward(streams, fn)`` and
``forward_tail(streams, fn, n_last)`` follow python/montlok/rdt/mhc.py:160-201:
mhc_prepare (coefficients + aggregate), ``fn`` once, mhc_combine. Only the
constrained (Sinkhorn) residual is built; ``MONTLOK_CPP_MHC=0`` switches the
module off.
"""

from __future__ import annotations

import torch
from torch import nn

from . import torch_path
from ._gate import backend_enabled, ext, require_gpu_inference
from .layers import RMSNormHIP

_FAMILY = "MONTLOK_CPP_MHC"


class ManifoldHyperConnectionHIP(nn.Module):
    def __init__(self, d_model: int, n_streams: int = 4, sinkhorn_iters: int = 20, constrain: bool = True,
                 rmsnorm_eps: float = 1e-5):
        super().__init__()
        if d_model <= 0:
            raise ValueError("d_model must be positive")
        if n_streams <= 0:
            raise ValueError("n_streams must be positive")
        if sinkhorn_iters < 0:
            raise ValueError("sinkhorn_iters must be non-negative")
        self.d_model = d_model
        self.n_streams = n_streams
        self.sinkhorn_iters = sinkhorn_iters
        self.constrain = constrain
        n = n_streams
        # Initial values of the upstream module: sigmoid(pre) = 1/n, 2 sigmoid(post) = 1, res ~ identity.
        pre_init = torch.full((n,), float(torch.log(torch.tensor(1.0 / (n - 1))))) if n > 1 else torch.full((1,), 20.0)
        self.pre_bias = nn.Parameter(pre_init)
        self.post_bias = nn.Parameter(torch.zeros(n))
        self.res_bias = nn.Parameter(torch.eye(n) * 3.0)
        self.dyn_norm = RMSNormHIP(d_model, eps=rmsnorm_eps)
        self.pre_proj = nn.Linear(d_model, n, bias=False)
        self.post_proj = nn.Linear(d_model, n, bias=False)
        self.res_proj = nn.Linear(d_model, n * n, bias=False)
        self.pre_alpha = nn.Parameter(torch.zeros(()))
        self.post_alpha = nn.Parameter(torch.zeros(()))
        self.res_alpha = nn.Parameter(torch.zeros(()))
        self._proj_w64_key = None
        self._proj_w64 = None

    # ------------------------------------------------------------ helpers
    def _check_streams(self, streams: torch.Tensor) -> None:
        if streams.ndim != 4:
            raise ValueError("streams must have shape [B, L, n_streams, d_model]")
        if streams.shape[-2] != self.n_streams:
            raise ValueError(f"expected n_streams={self.n_streams}, got {streams.shape[-2]}")
        if streams.shape[-1] != self.d_model:
            raise ValueError(f"expected d_model={self.d_model}, got {streams.shape[-1]}")

    def _require(self, streams: torch.Tensor) -> None:
        if not self.constrain:
            raise RuntimeError("ManifoldHyperConnectionHIP: only the Sinkhorn-constrained residual is built")
        require_gpu_inference(type(self).__name__, streams, _FAMILY)

    def _projection_block(self) -> torch.Tensor:
        """``cat(pre, post, res).weight`` in float64, cached per parameter version (mhc.py:48-60)."""
        weights = (self.pre_proj.weight, self.post_proj.weight, self.res_proj.weight)
        key = tuple((w.data_ptr(), w._version) for w in weights)
        if key != self._proj_w64_key:
            with torch.no_grad():
                self._proj_w64 = torch.cat(weights, 0).detach().to(torch.float64).contiguous()
            self._proj_w64_key = key
        return self._proj_w64

    def _prepare_args(self) -> tuple:
        return (self.dyn_norm.weight, self.dyn_norm.eps, self._projection_block(), self.pre_bias, self.post_bias,
                self.res_bias, self.pre_alpha, self.post_alpha, self.res_alpha, self.sinkhorn_iters)

    def _prepare(self, streams: torch.Tensor, *, allow_broadcast: bool = False, output_norm=None):
        if streams.ndim == 3:
            if not allow_broadcast:
                raise ValueError("broadcast streams are only valid at the start of a fused stage-2 pass")
            if streams.shape[-1] != self.d_model:
                raise ValueError(f"expected d_model={self.d_model}, got {streams.shape[-1]}")
            n_streams = self.n_streams
        else:
            self._check_streams(streams)
            n_streams = 0
        args = (streams, *self._prepare_args(), n_streams)
        if output_norm is not None:
            args += (output_norm.weight, output_norm.eps)
        return streams, ext().mhc_prepare(*args)

    def _combine(self, streams, prepared, out):
        _agg, _pre, post, res = prepared
        return ext().mhc_combine(streams, res, post, out.contiguous())

    def _combine_collapse(self, streams, prepared, out):
        _agg, _pre, post, res = prepared
        return ext().mhc_combine_collapse(streams, res, post, out.contiguous())

    def _combine_prepare(self, streams, prepared, out, next_hc, output_norm=None):
        """Write this residual and prepare ``next_hc`` in one pass (mhc.py:118-139)."""
        if not isinstance(next_hc, ManifoldHyperConnectionHIP):
            raise TypeError("next_hc must be a ManifoldHyperConnectionHIP")
        _agg, _pre, post, res = prepared
        args = (streams, res, post, out.contiguous(), *next_hc._prepare_args())
        if output_norm is not None:
            args += (output_norm.weight, output_norm.eps)
        new_streams, agg, pre, next_post, next_res = ext().mhc_combine_prepare(*args)
        return new_streams, (agg, pre, next_post, next_res)

    # ------------------------------------------------------------ public API
    def expand(self, x: torch.Tensor) -> torch.Tensor:
        """Replicate ``[B, L, d]`` into ``n`` streams ``[B, L, n, d]``."""
        if x.ndim != 3:
            raise ValueError("x must have shape [B, L, d_model]")
        if x.shape[-1] != self.d_model:
            raise ValueError(f"expected d_model={self.d_model}, got {x.shape[-1]}")
        return x.unsqueeze(-2).expand(-1, -1, self.n_streams, -1).contiguous()

    def collapse(self, streams: torch.Tensor) -> torch.Tensor:
        """Mean over the ``n`` streams, ``[B, L, n, d] -> [B, L, d]``."""
        self._check_streams(streams)
        return streams.mean(dim=-2)

    def forward(self, streams: torch.Tensor, fn) -> torch.Tensor:
        self._check_streams(streams)
        if not backend_enabled(_FAMILY):
            return torch_path.mhc_forward(self, streams, fn)
        self._require(streams)
        streams, prepared = self._prepare(streams)
        agg = prepared[0]
        out = fn(agg)
        if out.shape != agg.shape:
            raise ValueError("wrapped fn must preserve [B, L, d_model] shape")
        return self._combine(streams, prepared, out)

    def forward_tail(self, streams: torch.Tensor, fn, n_last: int = 1) -> torch.Tensor:
        """Residual output ``[B, n_last, n, d]`` of the trailing positions; ``fn`` sees the whole aggregate
        ``[B, L, d]`` and returns ``[B, n_last, d]``."""
        self._check_streams(streams)
        length = streams.shape[1]
        if not 1 <= n_last <= length:
            raise ValueError("n_last must be between 1 and the sequence length")
        if not backend_enabled(_FAMILY):
            return torch_path.mhc_forward(self, streams, fn, n_last)
        self._require(streams)
        streams, prepared = self._prepare(streams)
        agg, _pre, post, res = prepared
        out = fn(agg)
        if out.shape != (streams.shape[0], n_last, streams.shape[-1]):
            raise ValueError("wrapped fn must return [B, n_last, d_model]")
        tail = slice(length - n_last, length)
        return ext().mhc_combine(streams[:, tail].contiguous(), res[:, tail].contiguous(),
                                 post[:, tail].contiguous(), out.contiguous())


ManifoldHyperConnectionCPU = ManifoldHyperConnectionHIP

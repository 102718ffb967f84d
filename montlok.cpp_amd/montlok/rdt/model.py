"""Model-level drop-in on the ROCm device: ``RDT4QuantHIP`` / ``MultiAssetRDTHIP``
with the reference's names ``RDT4QuantCPU`` / ``MultiAssetRDTCPU``
(python/montlok/rdt/model.py:289-417).

The module tree is the upstream two-stage model's (Model/two_stage.py
``TwoStageCore`` and ``MHCAttnSubLayer``, Model/blocks.py ``MambaSubLayer``,
Model/layers/mamba3_layer.py ``Mamba3Layer``), built from this package's GPU
modules, so a checkpoint of the upstream model loads with
``load_state_dict(strict=True)`` under the same keys:

    projection.{weight,bias}, input_norm.{weight,bias}
    recurrent.stage1.<i>.mamba.norm.weight
    recurrent.stage1.<i>.mamba.mamba.{in_proj.weight, dt_bias, B_bias, C_bias,
        B_norm.weight, C_norm.weight, D, out_proj.weight}
    recurrent.stage1.<i>.ffn_norm.weight, recurrent.stage1.<i>.ffn.{w_in,w_down}.weight
    recurrent.stage2.<j>.{attn_norm, ffn_norm}.weight
    recurrent.stage2.<j>.attn.{q_proj, kv_down, kv_up, k_rope_proj, o_proj}.weight,
        recurrent.stage2.<j>.attn.kv_norm.{weight,bias}
    recurrent.stage2.<j>.ffn.{w_in,w_down}.weight
    recurrent.stage2.<j>.{attn_hc,ffn_hc}.{pre_bias, post_bias, res_bias, dyn_norm.weight,
        pre_proj.weight, post_proj.weight, res_proj.weight, pre_alpha, post_alpha, res_alpha}
    final_norm.weight, head.{weight,bias}

``forward`` follows the reference's tail path (model.py:340-364): stage 1 in one
native call (``stage1_forward``), then, for one stage-2 layer, the whole
recurrent tail in one call (``stage2_tail_forward``) that evaluates the last
position only; with several stage-2 layers the full recurrence runs and the
last position is taken (the same arithmetic row for row). Parameter packs are
cached per sequence length and device and dropped by ``load_state_dict`` and
``train`` (model.py:310-323). Configurations the reference sends to upstream
PyTorch instead of its kernels (other core types or drift modes, prelude/coda
blocks, morphological RoPE, mixture-of-LoRA FFNs, ACT) raise here.
"""

from __future__ import annotations

import dataclasses
import os
from typing import Any

import torch
from torch import nn
from torch.nn import functional as F

from ._gate import backend_enabled, ext, require_gpu_inference
from .linear import cpu_linear
from .layers import GroupedRMSNormHIP, LayerNormHIP, RMSNormHIP, SwiGLUHIP
from .mamba3 import Mamba3HIP, cpp_backend
from .mhc import ManifoldHyperConnectionHIP
from .mla import MLAHIP

_FAMILY = "MONTLOK_CPP_MODEL"


def tail_enabled() -> bool:
    """The last-position tail path (model.py:47-48); ``MONTLOK_CPP_TAIL=0`` runs the full recurrence over
    every position and takes the last row instead."""
    return cpp_backend() is not None and os.environ.get("MONTLOK_CPP_TAIL") != "0"


def native_stage1_enabled() -> bool:
    """Stage 1 as one ``stage1_forward`` call (model.py:51-55); ``MONTLOK_CPP_NATIVE_STAGE1=0`` (or
    ``MONTLOK_CPP_FUSED=0``) runs its sub-layer modules one by one."""
    return (os.environ.get("MONTLOK_CPP_NATIVE_STAGE1") != "0" and os.environ.get("MONTLOK_CPP_LAYERS") != "0"
            and cpp_backend() == "fused")


def native_stage2_enabled() -> bool:
    """The stage-2 tail as one ``stage2_tail_forward`` call (model.py:144-148); ``MONTLOK_CPP_NATIVE_STAGE2=0``
    runs the stage-2 modules one by one over every position."""
    return os.environ.get("MONTLOK_CPP_NATIVE_STAGE2") != "0" and os.environ.get("MONTLOK_CPP_LAYERS") != "0"


@dataclasses.dataclass
class RDTModelConfig:
    """The fields of the upstream ``RDTConfig`` (Model/config.py:94-300) that the two-stage mHC inference
    path reads, with the upstream defaults. Other keys of a checkpoint's ``model`` section (training,
    tokenizer and ablation settings) are accepted and kept in ``extra`` without effect."""

    d_model: int = 768
    n_heads: int = 12
    head_dim: int = 64
    kv_lora_rank: int = 256
    q_lora_rank: int = 0
    rope_head_dim: int = 32
    nope_head_dim: int = 32
    ffn_hidden: int = 2048
    n_prelude: int = 2
    n_coda: int = 2
    recurrent_steps: int = 8
    core_type: str = "interleaved"
    recurrent_drift_mode: str = "none"
    mhc_n_streams: int = 4
    mhc_sinkhorn_iters: int = 20
    stage1_mamba_layers: int = 5
    stage2_attn_layers: int = 1
    two_stage_downsample: bool = False
    use_act: bool = False
    use_mol: bool = False
    mamba_d_state: int = 128
    mamba_expand: int = 2
    mamba_headdim: int = 64
    mamba_dt_min: float = 0.001
    mamba_dt_max: float = 0.1
    mamba_dt_init_floor: float = 1e-4
    mamba_chunk_size: int = 64
    use_official_mamba: bool = True
    rope_theta: float = 10000.0
    use_morphological_rope: bool = True
    max_seq_len: int = 4096
    rmsnorm_eps: float = 1e-5
    extra: dict = dataclasses.field(default_factory=dict)

    @classmethod
    def from_dict(cls, values: dict[str, Any]) -> "RDTModelConfig":
        names = {f.name for f in dataclasses.fields(cls)} - {"extra"}
        cfg = cls(**{k: v for k, v in values.items() if k in names})
        cfg.extra = {k: v for k, v in values.items() if k not in names}
        cfg.validate()
        return cfg

    def validate(self) -> None:
        unsupported = [
            (self.core_type != "two_stage", f"core_type={self.core_type!r} (only 'two_stage')"),
            (self.recurrent_drift_mode != "mhc", f"recurrent_drift_mode={self.recurrent_drift_mode!r} (only 'mhc')"),
            (self.n_prelude != 0 or self.n_coda != 0, "prelude/coda blocks"),
            (self.use_morphological_rope, "morphological RoPE"),
            (self.use_mol, "mixture-of-LoRA FFNs"),
            (self.use_act, "adaptive computation time"),
            (self.two_stage_downsample, "two-stage downsampling"),
        ]
        for bad, what in unsupported:
            if bad:
                raise NotImplementedError(f"RDT4QuantHIP: {what} is not on the GPU path")
        if not self.use_official_mamba:
            raise ValueError("the CPU runtime requires a checkpoint trained with use_official_mamba=True")
        if self.rope_head_dim + self.nope_head_dim != self.head_dim:
            raise ValueError("rope_head_dim + nope_head_dim must equal head_dim")
        if self.stage1_mamba_layers <= 0 or self.stage2_attn_layers <= 0:
            raise ValueError("stage1_mamba_layers and stage2_attn_layers must be positive")
        if self.recurrent_steps <= 0:
            raise ValueError("recurrent_steps must be positive")


class Mamba3LayerHIP(nn.Module):
    """Model/layers/mamba3_layer.py ``Mamba3Layer`` with the official backend: x + mixer(GroupedRMSNorm(x))."""

    def __init__(self, cfg: RDTModelConfig, layer_idx: int | None = None, num_groups: int = 8):
        super().__init__()
        self.cfg = cfg
        self.layer_idx = layer_idx
        self.norm = GroupedRMSNormHIP(cfg.d_model, num_groups=num_groups, eps=cfg.rmsnorm_eps)
        self.mamba = Mamba3HIP(d_model=cfg.d_model, d_state=cfg.mamba_d_state, expand=cfg.mamba_expand,
                               headdim=cfg.mamba_headdim, chunk_size=cfg.mamba_chunk_size, dt_min=cfg.mamba_dt_min,
                               dt_max=cfg.mamba_dt_max, dt_init_floor=cfg.mamba_dt_init_floor, layer_idx=layer_idx)
        self.backend = "official"

    def forward(self, x: torch.Tensor, attn_mask: torch.Tensor | None = None, **_: Any) -> torch.Tensor:
        if attn_mask is not None:
            raise NotImplementedError("Mamba3LayerHIP: padding masks are not on the GPU path")
        if cpp_backend() != "fused":
            return x + self.mamba(self.norm(x))
        require_gpu_inference(type(self).__name__, x)
        m = self.mamba
        return ext().mamba3_block(x, self.norm.weight, self.norm.eps, self.norm.num_groups, m.in_proj.weight,
                                  m.out_proj.weight, *m._mixer_args(), *m._geometry())


class MambaSubLayerHIP(nn.Module):
    """Model/blocks.py ``MambaSubLayer``: Mamba layer, then x + SwiGLU(RMSNorm(x))."""

    def __init__(self, cfg: RDTModelConfig, layer_idx: int | None = None):
        super().__init__()
        self.layer_idx = layer_idx
        self.mamba = Mamba3LayerHIP(cfg, layer_idx=layer_idx)
        self.ffn_norm = RMSNormHIP(cfg.d_model, eps=cfg.rmsnorm_eps)
        self.ffn = SwiGLUHIP(cfg.d_model, cfg.ffn_hidden)

    def forward(self, x: torch.Tensor, attn_mask: torch.Tensor | None = None, **_: Any) -> torch.Tensor:
        x = self.mamba(x, attn_mask=attn_mask)
        return x + self.ffn(self.ffn_norm(x))


class _MLAConfigView:
    """The attribute view ``MLAHIP`` reads (the upstream MLA takes the whole RDTConfig)."""

    def __init__(self, cfg: RDTModelConfig):
        self.d_model, self.n_heads, self.head_dim = cfg.d_model, cfg.n_heads, cfg.head_dim
        self.nope_head_dim, self.rope_head_dim = cfg.nope_head_dim, cfg.rope_head_dim
        self.kv_lora_rank, self.q_lora_rank, self.rope_theta = cfg.kv_lora_rank, cfg.q_lora_rank, cfg.rope_theta
        self.max_seq_len, self.use_morphological_rope = cfg.max_seq_len, cfg.use_morphological_rope


class MHCAttnSubLayerHIP(nn.Module):
    """Model/two_stage.py ``MHCAttnSubLayer``: the attention and FFN residuals, each through its own mHC."""

    def __init__(self, cfg: RDTModelConfig, layer_idx: int | None = None):
        super().__init__()
        self.layer_idx = layer_idx
        self.attn_norm = RMSNormHIP(cfg.d_model, eps=cfg.rmsnorm_eps)
        self.attn = MLAHIP(_MLAConfigView(cfg))
        self.ffn_norm = RMSNormHIP(cfg.d_model, eps=cfg.rmsnorm_eps)
        self.ffn = SwiGLUHIP(cfg.d_model, cfg.ffn_hidden)
        self.attn_hc = ManifoldHyperConnectionHIP(cfg.d_model, n_streams=cfg.mhc_n_streams,
                                                  sinkhorn_iters=cfg.mhc_sinkhorn_iters)
        self.ffn_hc = ManifoldHyperConnectionHIP(cfg.d_model, n_streams=cfg.mhc_n_streams,
                                                 sinkhorn_iters=cfg.mhc_sinkhorn_iters)

    def forward(self, streams: torch.Tensor, **_: Any) -> torch.Tensor:
        streams = self.attn_hc(streams, lambda inp: self.attn(self.attn_norm(inp)))
        return self.ffn_hc(streams, lambda inp: self.ffn(self.ffn_norm(inp)))


class TwoStageCoreHIP(nn.Module):
    """Model/two_stage.py ``TwoStageCore`` in the mHC drift mode (inference): stage 1 (Mamba sub-layers),
    expand to n streams, ``steps`` passes of stage 2, collapse."""

    def __init__(self, cfg: RDTModelConfig):
        super().__init__()
        self.cfg = cfg
        self.drift_mode = cfg.recurrent_drift_mode
        self.n_streams = cfg.mhc_n_streams
        self.stage1 = nn.ModuleList(MambaSubLayerHIP(cfg, layer_idx=i) for i in range(cfg.stage1_mamba_layers))
        self.stage2 = nn.ModuleList(MHCAttnSubLayerHIP(cfg, layer_idx=i) for i in range(cfg.stage2_attn_layers))
        self.boundary_norm = None

    def _check_inputs(self, e0: torch.Tensor) -> None:
        if e0.ndim != 3:
            raise ValueError("e0 must have shape [B, L, d_model]")
        if e0.shape[-1] != self.cfg.d_model:
            raise ValueError(f"expected d_model={self.cfg.d_model}, got {e0.shape[-1]}")

    def _stage1_packs(self) -> list:
        packs = self.__dict__.get("_montlok_stage1_parameter_pack")
        if packs is None or os.environ.get("MONTLOK_CACHE_PARAMETER_PACKS") == "0":
            packs = []
            for layer in self.stage1:
                mixer, ffn = layer.mamba.mamba, layer.ffn
                empty = mixer.D.new_empty(0)
                packs.append((layer.mamba.norm.weight, mixer.in_proj.weight, mixer.out_proj.weight, mixer.B_bias,
                              mixer.C_bias, mixer.B_norm.weight, mixer.C_norm.weight, mixer.dt_bias, mixer.D,
                              layer.ffn_norm.weight, ffn.w_in.weight,
                              ffn.w_in.bias if ffn.w_in.bias is not None else empty, ffn.w_down.weight,
                              ffn.w_down.bias if ffn.w_down.bias is not None else empty))
            if os.environ.get("MONTLOK_CACHE_PARAMETER_PACKS") != "0":
                self.__dict__["_montlok_stage1_parameter_pack"] = packs
        return packs

    def run_stage1(self, e0: torch.Tensor) -> torch.Tensor:
        """All stage-1 sub-layers in one native call (model.py:67-113)."""
        first = self.stage1[0]
        mixer = first.mamba.mamba
        return ext().stage1_forward(e0, self._stage1_packs(), first.mamba.norm.eps, first.mamba.norm.num_groups,
                                    first.ffn_norm.eps, mixer.d_state, mixer.num_bc_heads, mixer.nheads,
                                    mixer.headdim, mixer.num_rope_angles, mixer.B_norm.eps, mixer.C_norm.eps,
                                    mixer.A_floor)

    def run_stage1_modules(self, e0: torch.Tensor) -> torch.Tensor:
        """Stage 1 sub-layer by sub-layer (``core._run_stage1``, the reference's path without the native
        stage-1 call)."""
        x = e0
        for layer in self.stage1:
            x = layer(x)
        return x

    def _expand(self, x: torch.Tensor) -> torch.Tensor:
        return x.unsqueeze(-2).expand(-1, -1, self.n_streams, -1).contiguous()

    def _collapse(self, streams: torch.Tensor) -> torch.Tensor:
        return streams.mean(dim=-2)

    def forward(self, e0: torch.Tensor, steps: int | None = None, **_: Any) -> tuple[torch.Tensor, dict]:
        self._check_inputs(e0)
        total = int(steps if steps is not None else self.cfg.recurrent_steps)
        if total <= 0:
            raise ValueError("steps must be positive")
        backbone = self.run_stage1(e0) if native_stage1_enabled() else self.run_stage1_modules(e0)
        streams = self._expand(backbone)
        for _step in range(total):
            for layer in self.stage2:
                streams = layer(streams)
        return self._collapse(streams), {"steps_used": total, "ponder_cost": e0.new_tensor(0.0),
                                         "global_semantic": backbone.mean(dim=1)}

    def _stage2_packs(self, layer: MHCAttnSubLayerHIP, length: int, device) -> tuple:
        key = (length, device.type, device.index)
        cache = layer.__dict__.get("_montlok_stage2_parameter_packs")
        packed = None if cache is None else cache.get(key)
        if packed is None or os.environ.get("MONTLOK_CACHE_PARAMETER_PACKS") == "0":
            attn, ffn = layer.attn, layer.ffn

            def hc_pack(hc):
                return (hc.dyn_norm.weight, hc._projection_block(), hc.pre_bias, hc.post_bias, hc.res_bias,
                        hc.pre_alpha, hc.post_alpha, hc.res_alpha)

            empty = attn.kv_up.weight.new_empty(0, dtype=torch.float32)
            cos, sin = attn._rope_tables(length, 0, device)
            packed = (hc_pack(layer.attn_hc),
                      (attn._in_proj_weight(True), attn._in_proj_weight(False), attn.q_proj.weight,
                       attn.kv_norm.weight, attn.kv_norm.bias if attn.kv_norm.bias is not None else empty,
                       attn.kv_up.weight, attn.o_proj.weight, cos, sin),
                      hc_pack(layer.ffn_hc),
                      (ffn.w_in.weight, ffn.w_in.bias if ffn.w_in.bias is not None else empty, ffn.w_down.weight,
                       ffn.w_down.bias if ffn.w_down.bias is not None else empty))
            if os.environ.get("MONTLOK_CACHE_PARAMETER_PACKS") != "0":
                if cache is None:
                    cache = {}
                    layer.__dict__["_montlok_stage2_parameter_packs"] = cache
                cache[key] = packed
        return packed

    def stage2_tail(self, backbone: torch.Tensor, depth: int) -> torch.Tensor:
        """Hidden state [B, 1, d] of the last position after ``depth`` passes of the single stage-2 layer,
        in one native call (model.py:160-232)."""
        layer = self.stage2[0]
        attn_hc, mla, ffn_hc, ffn = self._stage2_packs(layer, backbone.shape[1], backbone.device)
        a = layer.attn
        return ext().stage2_tail_forward(backbone, depth, layer.attn_hc.n_streams, attn_hc, layer.attn_hc.dyn_norm.eps,
                                         layer.attn_hc.sinkhorn_iters, layer.attn_norm.weight, layer.attn_norm.eps,
                                         mla, a.kv_norm.eps, a.n_heads, a.head_dim, a.nope_dim, a.kv_lora_rank,
                                         a.scale, ffn_hc, layer.ffn_hc.dyn_norm.eps, layer.ffn_hc.sinkhorn_iters,
                                         layer.ffn_norm.weight, layer.ffn_norm.eps, ffn)

    def clear_parameter_packs(self) -> None:
        self.__dict__.pop("_montlok_stage1_parameter_pack", None)
        for layer in self.stage2:
            layer.__dict__.pop("_montlok_stage2_parameter_packs", None)


class RDT4QuantHIP(nn.Module):
    """python/montlok/rdt/model.py:289-390 on the ROCm device: features -> projection -> LayerNorm ->
    two-stage mHC core -> RMSNorm of the last position -> quantile head (low, median, high per horizon)."""

    def __init__(self, n_features: int, config: dict):
        super().__init__()
        self.cfg = RDTModelConfig.from_dict(config["model"])
        d = self.cfg.d_model
        self.projection = nn.Linear(n_features, d)
        self.input_norm = LayerNormHIP(d)
        self.prelude, self.coda = nn.ModuleList(), nn.ModuleList()
        self.recurrent = TwoStageCoreHIP(self.cfg)
        self.final_norm = RMSNormHIP(d, eps=self.cfg.rmsnorm_eps)
        self.head = nn.Linear(d, len(config["horizons_minutes"]) * 3)
        self.n_horizons = len(config["horizons_minutes"])

    def load_state_dict(self, state_dict, strict: bool = True, assign: bool = False):
        result = super().load_state_dict(state_dict, strict=strict, assign=assign)
        self.recurrent.clear_parameter_packs()
        return result

    def train(self, mode: bool = True):
        result = super().train(mode)
        self.recurrent.clear_parameter_packs()
        return result

    def _embed(self, inputs: torch.Tensor) -> torch.Tensor:
        x = inputs.float()
        if backend_enabled():
            require_gpu_inference(type(self).__name__, x, _FAMILY)
        return self.input_norm(cpu_linear(x, self.projection.weight, self.projection.bias))

    def encode(self, inputs: torch.Tensor, depth: int):
        """Hidden states of every position after ``depth`` stage-2 passes, and the core's info dict."""
        return self.recurrent(self._embed(inputs), steps=depth)

    def _hidden_tail(self, embedded: torch.Tensor, depth: int) -> torch.Tensor:
        core = self.recurrent
        core._check_inputs(embedded)
        depth = int(depth)
        if depth <= 0:
            raise ValueError("steps must be positive")
        backbone = core.run_stage1(embedded) if native_stage1_enabled() else core.run_stage1_modules(embedded)
        if len(core.stage2) == 1 and native_stage2_enabled():
            return core.stage2_tail(backbone, depth)
        streams = core._expand(backbone)
        for _ in range(depth):
            for layer in core.stage2:
                streams = layer(streams)
        return core._collapse(streams)[:, -1:]

    @staticmethod
    def _quantiles(raw: torch.Tensor) -> torch.Tensor:
        center = raw[..., 0]
        return torch.stack((center - F.softplus(raw[..., 1]), center, center + F.softplus(raw[..., 2])), dim=-1)

    def _head(self, hidden: torch.Tensor, head: nn.Linear, rows: int) -> torch.Tensor:
        last = self.final_norm(hidden[:, -1].contiguous())
        return self._quantiles(cpu_linear(last, head.weight, head.bias).reshape(-1, rows, 3))

    def _hidden_for_head(self, embedded: torch.Tensor, depth: int) -> torch.Tensor:
        """model.py:366-370: the tail path, or (``MONTLOK_CPP_TAIL=0``) the full recurrence's hidden states."""
        if tail_enabled():
            return self._hidden_tail(embedded, depth)
        hidden, _ = self.recurrent(embedded, steps=depth)
        return hidden

    def forward(self, inputs: torch.Tensor, depth: int):
        hidden = self._hidden_for_head(self._embed(inputs), depth)
        return self._head(hidden, self.head, self.n_horizons), hidden.detach().float().square().mean().sqrt()


class MultiAssetRDTHIP(RDT4QuantHIP):
    """python/montlok/rdt/model.py:393-417: the crypto model plus typed stock inputs (their own projection,
    LayerNorm, asset and period embeddings, and one 3 x 3 quantile head per stock domain)."""

    def __init__(self, base_config: dict, asset_count: int):
        super().__init__(57, base_config)
        d = self.cfg.d_model
        self.stock_projection = nn.Linear(23, d)
        self.stock_norm = LayerNormHIP(d)
        self.asset_embedding = nn.Embedding(asset_count, d)
        self.period_embedding = nn.Embedding(2, d)
        self.stock_heads = nn.ModuleDict({name: nn.Linear(d, 9) for name in ("equity_daily", "token_hour")})

    def forward(self, inputs: torch.Tensor, depth: int, domain: str = "crypto", asset_id=None):
        if domain == "crypto":
            return super().forward(inputs, depth)
        if domain not in self.stock_heads or asset_id is None:
            raise ValueError("typed stock domain and asset identifiers are required")
        x = inputs.float()
        if backend_enabled():
            require_gpu_inference(type(self).__name__, x, _FAMILY)
        identity = self.asset_embedding(asset_id)
        period = self.period_embedding.weight[0 if domain == "equity_daily" else 1]
        projected = cpu_linear(x, self.stock_projection.weight, self.stock_projection.bias)
        embedded = self.stock_norm(projected + identity[:, None] + period)
        hidden = self._hidden_for_head(embedded, depth)
        return self._head(hidden, self.stock_heads[domain], 3), hidden.detach().float().square().mean().sqrt()


# The reference's class names, for code that imports them.
RDT4QuantCPU = RDT4QuantHIP
MultiAssetRDTCPU = MultiAssetRDTHIP

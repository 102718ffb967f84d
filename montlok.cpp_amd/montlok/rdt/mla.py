"""Multi-head latent attention (MLA) forward on the GPU.

``MLAHIP`` (also importable as ``MLACPU``) is built from the same config object
as the upstream module and has its parameters (reference/Model/layers/
mla.py:15-76): ``q_proj`` (or ``q_down``/``q_norm``/``q_up`` when
q_lora_rank > 0), ``kv_down``, ``kv_norm``, ``kv_up``, ``k_rope_proj``,
``o_proj``. ``forward`` (full causal sequence) and ``forward_last`` (trailing
positions) follow python/montlok/rdt/mla.py:131-214: one stacked input GEMM
over [q_proj; kv_down; k_rope_proj], latent LayerNorm, kv_up, RoPE on the
rotate_half halves, attention with the reference's mask conventions, o_proj.
RoPE tables are built with torch on the CPU exactly as the upstream
token-index RoPE does (rope.py:9-16, 138-166) and cached per device. With bf16
weights the attention contractions also run on bf16 matrix cores.
KV caches, padding masks and morphological RoPE are not built.
"""

from __future__ import annotations

import math

import torch
from torch import nn

from . import torch_path
from ._gate import backend_enabled, ext, require_gpu_inference

_FAMILY = "MONTLOK_CPP_LAYERS"


def _build_freqs(dim: int, theta: float) -> torch.Tensor:
    idx = torch.arange(0, dim, 2, dtype=torch.float32)
    return 1.0 / (theta ** (idx / dim))


def rope_tables(seq_len: int, rope_dim: int, theta: float = 10000.0, pos_offset: int = 0):
    """Token-index cos/sin ``[seq_len, rope_dim]`` (cat(angles, angles)), computed on the CPU in fp32."""
    freqs = _build_freqs(rope_dim, theta)
    pos = torch.arange(pos_offset, pos_offset + seq_len, dtype=torch.float32)
    angles = pos.unsqueeze(-1) * freqs.unsqueeze(0)
    emb = torch.cat([angles, angles], dim=-1)
    return emb.cos(), emb.sin()


class TokenRoPE(nn.Module):
    """The non-morphological RoPE of the upstream module: a non-persistent ``freqs`` buffer."""

    def __init__(self, rope_dim: int, theta: float = 10000.0, **_: object):
        super().__init__()
        if rope_dim <= 0 or rope_dim % 2:
            raise ValueError("rope_dim must be positive and even")
        self.rope_dim = rope_dim
        self.theta = theta
        self.register_buffer("freqs", _build_freqs(rope_dim, theta), persistent=False)


class MLAHIP(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.cfg = cfg
        self.d_model = cfg.d_model
        self.n_heads = cfg.n_heads
        self.head_dim = cfg.head_dim
        self.nope_dim = cfg.nope_head_dim
        self.rope_dim = cfg.rope_head_dim
        self.kv_lora_rank = cfg.kv_lora_rank
        self.q_lora_rank = getattr(cfg, "q_lora_rank", 0)
        self.dropout = getattr(cfg, "dropout", 0.0)
        if getattr(cfg, "use_morphological_rope", False):
            raise ValueError("morphological RoPE is not built for the GPU path")
        if self.head_dim != self.nope_dim + self.rope_dim:
            raise ValueError("head_dim must equal nope_head_dim + rope_head_dim")
        if self.d_model != self.n_heads * self.head_dim:
            raise ValueError("d_model must equal n_heads * head_dim")
        if self.rope_dim % 2 != 0:
            raise ValueError("rope_head_dim must be even")
        if self.kv_lora_rank <= 0:
            raise ValueError("kv_lora_rank must be positive")
        if self.q_lora_rank < 0:
            raise ValueError("q_lora_rank must be non-negative")
        hd = self.n_heads * self.head_dim
        if self.q_lora_rank > 0:
            self.q_down = nn.Linear(self.d_model, self.q_lora_rank, bias=False)
            self.q_norm = nn.LayerNorm(self.q_lora_rank)
            self.q_up = nn.Linear(self.q_lora_rank, hd, bias=False)
        else:
            self.q_proj = nn.Linear(self.d_model, hd, bias=False)
        self.kv_down = nn.Linear(self.d_model, self.kv_lora_rank, bias=False)
        self.kv_norm = nn.LayerNorm(self.kv_lora_rank)
        self.kv_up = nn.Linear(self.kv_lora_rank, self.n_heads * (self.nope_dim + self.head_dim), bias=False)
        self.k_rope_proj = nn.Linear(self.d_model, self.rope_dim, bias=False)
        self.o_proj = nn.Linear(hd, self.d_model, bias=False)
        self.rope = TokenRoPE(self.rope_dim, theta=getattr(cfg, "rope_theta", 10000.0))
        self.scale = 1.0 / math.sqrt(self.head_dim)
        self._rope_cache: dict = {}
        self._in_proj_cache: dict = {}

    def _in_proj_weight(self, with_q: bool) -> torch.Tensor:
        """``[q_proj;] kv_down; k_rope_proj`` stacked, cached per parameter version (mla.py:54-73)."""
        weights = (self.kv_down.weight, self.k_rope_proj.weight)
        if with_q:
            weights = (self.q_proj.weight, *weights)
        key = tuple((w.data_ptr(), w._version) for w in weights)
        cached = self._in_proj_cache.get(with_q)
        if cached is None or cached[0] != key:
            with torch.no_grad():
                cached = (key, torch.cat(weights, 0).detach().contiguous())
            self._in_proj_cache[with_q] = cached
        return cached[1]

    def _rope_tables(self, seq_len: int, pos_offset: int, device):
        key = (seq_len, pos_offset, str(device))
        tables = self._rope_cache.get(key)
        if tables is None:
            cos, sin = rope_tables(seq_len, self.rope_dim, self.rope.theta, pos_offset)
            tables = (cos.to(device), sin.to(device))
            if len(self._rope_cache) > 8:
                self._rope_cache.clear()
            self._rope_cache[key] = tables
        return tables

    def _check(self, x, word_pos=None, morph_depth=None, attn_mask=None, cache=None) -> None:
        if cache is not None or attn_mask is not None or word_pos is not None or morph_depth is not None:
            raise RuntimeError("MLAHIP: KV caches, attention masks and morphological positions are not built")
        if self.training:
            raise RuntimeError("MLAHIP: inference only (call .eval())")
        require_gpu_inference(type(self).__name__, x, _FAMILY)

    def forward(self, x: torch.Tensor, word_pos=None, morph_depth=None, attn_mask=None, causal: bool = True,
                cache=None, pos_offset: int = 0) -> torch.Tensor:
        if not backend_enabled(_FAMILY) and cache is None and attn_mask is None and word_pos is None and \
                morph_depth is None:
            return self._torch_forward(x, x.shape[1], causal, pos_offset)
        self._check(x, word_pos, morph_depth, attn_mask, cache)
        return self._attend(x, x.shape[1], causal, pos_offset)

    def _torch_forward(self, x: torch.Tensor, n_last: int, causal: bool, pos_offset: int) -> torch.Tensor:
        """``MONTLOK_CPP_LAYERS=0`` / ``MONTLOK_CPP=0``: the upstream PyTorch forward (``torch_path``)."""
        cos, sin = self._rope_tables(x.shape[1], pos_offset, x.device)
        return torch_path.mla_forward(self, x, cos, sin, n_last, causal)

    def forward_last(self, x: torch.Tensor, n_last: int = 1, pos_offset: int = 0) -> torch.Tensor:
        """Causal attention output ``[B, n_last, d_model]`` of the trailing positions."""
        if x.ndim != 3:
            raise ValueError("x must have shape [B, L, d_model]")
        if not 1 <= n_last <= x.shape[1]:
            raise ValueError("n_last must be between 1 and the sequence length")
        if not backend_enabled(_FAMILY):
            return self._torch_forward(x, n_last, True, pos_offset)
        self._check(x)
        return self._attend(x, n_last, True, pos_offset)

    def _project_q_rows(self, x_rows: torch.Tensor) -> torch.Tensor:
        c = ext()
        if self.q_lora_rank > 0:
            down = c.linear(x_rows, self.q_down.weight)
            return c.linear(c.layer_norm(down, self.q_norm.weight, self.q_norm.bias, self.q_norm.eps), self.q_up.weight)
        return c.linear(x_rows, self.q_proj.weight)

    def _attend(self, x: torch.Tensor, n_last: int, causal: bool, pos_offset: int) -> torch.Tensor:
        bsz, seq_len, dim = x.shape
        if dim != self.d_model:
            raise ValueError(f"expected d_model={self.d_model}, got {dim}")
        c = ext()
        fuse_q = self.q_lora_rank == 0 and n_last == seq_len
        cos, sin = self._rope_tables(seq_len, pos_offset, x.device)
        if self.q_lora_rank == 0 and n_last in (1, seq_len):
            q_weight = self.q_proj.weight if n_last == 1 else x.new_empty(0)
            return c.mla_forward(x, self._in_proj_weight(fuse_q), q_weight, self.kv_norm.weight, self.kv_norm.bias,
                                 self.kv_norm.eps, self.kv_up.weight, self.o_proj.weight, cos, sin, self.n_heads,
                                 self.head_dim, self.nope_dim, self.kv_lora_rank, n_last, causal, self.scale)
        projected = c.linear(x, self._in_proj_weight(fuse_q))
        q_width = self.n_heads * self.head_dim if fuse_q else 0
        if fuse_q:
            q = projected[..., :q_width].unflatten(-1, (self.n_heads, self.head_dim))
        else:
            q = self._project_q_rows(x[:, seq_len - n_last:].contiguous()).view(bsz, n_last, self.n_heads,
                                                                                self.head_dim)
        kv_latent = projected[..., q_width:q_width + self.kv_lora_rank]
        k_rope = projected[..., q_width + self.kv_lora_rank:]
        kv = c.linear(c.layer_norm(kv_latent, self.kv_norm.weight, self.kv_norm.bias, self.kv_norm.eps),
                      self.kv_up.weight).view(bsz, seq_len, self.n_heads, self.nope_dim + self.head_dim)
        k = c.mla_rope_qk(q, kv, k_rope, cos, sin, self.nope_dim)
        v = kv[..., self.nope_dim:]
        if n_last == seq_len:
            mask = c.MASK_CAUSAL_TOP_LEFT if causal else c.MASK_NONE
        elif n_last == 1 or not causal:
            mask = c.MASK_NONE
        else:
            mask = c.MASK_CAUSAL_BOTTOM_RIGHT
        precision = torch.bfloat16 if self.o_proj.weight.dtype == torch.bfloat16 else torch.float32
        out = c.attention(q, k, v, mask, self.scale, precision).view(bsz, n_last, self.d_model)
        return c.linear(out, self.o_proj.weight)


MLACPU = MLAHIP

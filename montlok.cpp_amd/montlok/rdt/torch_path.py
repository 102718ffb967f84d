"""The upstream PyTorch forward of each drop-in module: the reference's A/B ladder.

The reference runs its upstream PyTorch modules where its kernels are switched
off (README.md:268-271): ``MONTLOK_CPP=0`` for every module (and the pure
PyTorch quadratic Mamba-3 of python/montlok/rdt/mamba3.py:199-256),
``MONTLOK_CPP_MHC=0`` for the hyper-connections (mhc.py:36-37, 62-69),
``MONTLOK_CPP_LAYERS=0`` for RMSNorm / LayerNorm / SwiGLU and MLA
(layers.py:32-39, mla.py:44-45). The drop-in modules of this package call the
functions below in exactly those cases, on whatever device the input is on, so
a mismatch can be bisected by switching one family at a time. These are plain
tensor programs of the upstream formulas (reference/Model/layers/rmsnorm.py,
swiglu.py, mhc.py, mla.py, rope.py and the quadratic Mamba-3 form), not the
kernels' arithmetic: they agree with the kernels to the reference's own
tolerances, not bit for bit. Only an explicit switch selects them; with the
switches on, a module that cannot take its kernel raises instead.
"""

from __future__ import annotations

import math

import torch
from torch.nn import functional as F


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, groups: int = 1) -> torch.Tensor:
    """RMSNorm / GroupedRMSNorm (reference/Model/layers/rmsnorm.py:21-28, 49-60): statistics in fp32."""
    shape = x.shape
    y = x.float().reshape(*shape[:-1], groups, shape[-1] // groups)
    y = (y * torch.rsqrt(y.pow(2).mean(dim=-1, keepdim=True) + eps)).reshape(shape)
    return y.to(x.dtype) * weight.to(x.dtype)


def swiglu(x: torch.Tensor, w_in: torch.nn.Linear, w_down: torch.nn.Linear) -> torch.Tensor:
    """w_down(silu(gate) * up), [gate | up] = w_in(x) (reference/Model/layers/swiglu.py:24-35)."""
    gate, up = F.linear(x, w_in.weight.to(x.dtype), _maybe(w_in.bias, x)).chunk(2, dim=-1)
    return F.linear(F.silu(gate) * up, w_down.weight.to(x.dtype), _maybe(w_down.bias, x))


def _maybe(bias, x):
    return None if bias is None else bias.to(x.dtype)


def _linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    return F.linear(x, weight.to(x.dtype))


# ------------------------------------------------------------------ mHC


def sinkhorn_knopp(log_alpha: torch.Tensor, n_iters: int) -> torch.Tensor:
    """Log-space Sinkhorn in fp32, row then column normalisation, at least one pass
    (reference/Model/layers/mhc.py:38-72)."""
    work = log_alpha.float()
    for _ in range(max(n_iters, 1)):
        work = work - torch.logsumexp(work, dim=-1, keepdim=True)
        work = work - torch.logsumexp(work, dim=-2, keepdim=True)
    return torch.exp(work).to(log_alpha.dtype)


def mhc_coefficients(hc, streams: torch.Tensor):
    """(pre [B,L,n], post [B,L,n], res [B,L,n,n]) of a ManifoldHyperConnection module from the stream
    mean's RMSNorm (mhc.py:151-196): sigmoid, 2 sigmoid and Sinkhorn (softplus when unconstrained)."""
    ref = rms_norm(streams.mean(dim=-2), hc.dyn_norm.weight, hc.dyn_norm.eps)
    n = hc.n_streams
    pre = torch.sigmoid(hc.pre_bias + hc.pre_alpha * torch.tanh(_linear(ref, hc.pre_proj.weight)))
    post = 2.0 * torch.sigmoid(hc.post_bias + hc.post_alpha * torch.tanh(_linear(ref, hc.post_proj.weight)))
    logits = hc.res_bias + (hc.res_alpha * torch.tanh(_linear(ref, hc.res_proj.weight))).view(*ref.shape[:-1], n, n)
    res = sinkhorn_knopp(logits, hc.sinkhorn_iters) if hc.constrain else F.softplus(logits)
    return pre.to(streams.dtype), post.to(streams.dtype), res.to(streams.dtype)


def mhc_forward(hc, streams: torch.Tensor, fn, n_last: int | None = None) -> torch.Tensor:
    """agg = sum_i pre_i s_i; out = fn(agg); new = res @ streams + post (x) out (mhc.py:198-218); with
    ``n_last`` only the trailing positions are written (fn returns [B, n_last, d])."""
    pre, post, res = mhc_coefficients(hc, streams)
    agg = torch.einsum("bln,blnd->bld", pre, streams)
    out = fn(agg)
    if n_last is not None:
        tail = slice(streams.shape[1] - n_last, streams.shape[1])
        streams, post, res = streams[:, tail], post[:, tail], res[:, tail]
    if out.shape != (*streams.shape[:2], streams.shape[-1]):
        raise ValueError("wrapped fn must preserve [B, L, d_model] shape")
    return torch.einsum("blij,bljd->blid", res, streams) + post.unsqueeze(-1) * out.unsqueeze(-2)


# ------------------------------------------------------------------ MLA


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def mla_forward(m, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, n_last: int, causal: bool) -> torch.Tensor:
    """The upstream MLA forward (reference/Model/layers/mla.py:76-150, rope.py:18-38): q from q_proj (or
    q_down, q_norm, q_up), kv = kv_up(LayerNorm(kv_down(x))), k = cat(k_nope, rope(k_rope_proj(x))), q's rope
    dims rotated, scaled-dot-product attention (causal, bottom-right for trailing queries), o_proj; the
    output rows of the last ``n_last`` positions."""
    bsz, seq_len, _ = x.shape
    H, hd, nope = m.n_heads, m.head_dim, m.nope_dim
    if m.q_lora_rank > 0:
        down = _linear(x, m.q_down.weight)
        q = _linear(F.layer_norm(down, (m.q_lora_rank,), m.q_norm.weight, m.q_norm.bias, m.q_norm.eps), m.q_up.weight)
    else:
        q = _linear(x, m.q_proj.weight)
    q = q.view(bsz, seq_len, H, hd).transpose(1, 2)
    latent = F.layer_norm(_linear(x, m.kv_down.weight), (m.kv_lora_rank,), m.kv_norm.weight, m.kv_norm.bias,
                          m.kv_norm.eps)
    kv = _linear(latent, m.kv_up.weight).view(bsz, seq_len, H, nope + hd).transpose(1, 2)
    k_nope, v = kv.split([nope, hd], dim=-1)
    k_rope = _linear(x, m.k_rope_proj.weight).unsqueeze(1).expand(bsz, H, seq_len, m.rope_dim)
    c, s = cos.to(x.dtype)[None, None], sin.to(x.dtype)[None, None]
    q = torch.cat([q[..., :nope], q[..., nope:] * c + _rotate_half(q[..., nope:]) * s], dim=-1)
    k = torch.cat([k_nope, k_rope * c + _rotate_half(k_rope) * s], dim=-1)
    q = q[:, :, seq_len - n_last:]
    if causal:
        rows = torch.arange(n_last, device=x.device).unsqueeze(-1) + (seq_len - n_last)
        allow = torch.arange(seq_len, device=x.device).unsqueeze(0) <= rows
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=allow, scale=m.scale)
    else:
        out = F.scaled_dot_product_attention(q, k, v, scale=m.scale)
    return _linear(out.transpose(1, 2).reshape(bsz, n_last, H * hd), m.o_proj.weight)


# ------------------------------------------------------------------ Mamba-3


def _segment_sum(x: torch.Tensor) -> torch.Tensor:
    """out[..., t, s] = sum_{s < r <= t} x[..., r] for s <= t, -inf above the diagonal: a cumulative sum
    down each column of the strictly lower part (no difference of two running sums to cancel)."""
    length = x.shape[-1]
    ones = torch.ones(length, length, dtype=torch.bool, device=x.device)
    terms = x.unsqueeze(-1).expand(*x.shape, length).masked_fill(~torch.tril(ones, diagonal=-1), 0)
    return torch.cumsum(terms, dim=-2).masked_fill(~torch.tril(ones), -math.inf)


def mamba3_mixer(m, projected: torch.Tensor) -> torch.Tensor:
    """The Mamba-3 SISO mixer from the in_proj rows [B, L, W] to the gated output [B, L, d_inner], in the
    quadratic (segment-sum) form of python/montlok/rdt/mamba3.py:199-256: BCNorm'd B and C plus the per-head
    biases, dt = softplus(dt + dt_bias), adt = -max(heavy_tail(A), A_floor) dt, the rotary phase
    cumsum(tanh(angles) pi dt) wrapped to [0, 2 pi) applied to the pairs (2r, 2r + 1) of q and k, the
    trapezoid weights dt trap + dt_next (1 - trap_next), and the skip and gate terms."""
    B, L, _ = projected.shape
    H, N, G, D, R = m.nheads, m.d_state, m.num_bc_heads, m.headdim, m.num_rope_angles
    z, x, b_val, c_val, raw_dt, raw_a, raw_trap, raw_ang = torch.split(
        projected.float(), [m.d_inner, m.d_inner, N * G, N * G, H, H, H, R], dim=-1)
    z = z.reshape(B, L, H, D)
    x = x.reshape(B, L, H, D)

    def bc(value, norm, bias):
        v = rms_norm(value.reshape(B, L, G, N), norm.weight, norm.eps)
        return (v.unsqueeze(3) + bias.view(1, 1, G, H // G, N)).reshape(B, L, H, N)

    k_plain = bc(b_val, m.B_norm, m.B_bias)
    q_plain = bc(c_val, m.C_norm, m.C_bias)
    dt = F.softplus(raw_dt + m.dt_bias)
    a_val = -(raw_a.clamp_min(0) + torch.reciprocal(1 - raw_a.clamp_max(0))).clamp_min(m.A_floor)
    adt = a_val * dt
    q, k = q_plain, k_plain
    if R > 0:
        phase = torch.cumsum(torch.tanh(raw_ang).unsqueeze(2) * math.pi * dt.unsqueeze(-1), dim=1)
        phase = phase - 2 * math.pi * torch.floor(phase / (2 * math.pi))
        cos, sin = torch.cos(phase), torch.sin(phase)

        def rotate(v):
            pairs = v[..., :2 * R].unflatten(-1, (R, 2))
            left, right = pairs[..., 0], pairs[..., 1]
            turned = torch.stack((left * cos - right * sin, left * sin + right * cos), dim=-1).flatten(-2)
            return torch.cat((turned, v[..., 2 * R:]), dim=-1)

        q, k = rotate(q_plain), rotate(k_plain)
    trap = torch.sigmoid(raw_trap)
    dt_next = F.pad(dt[:, 1:], (0, 0, 0, 1))
    trap_next = F.pad(trap[:, 1:], (0, 0, 0, 1))
    gamma_next = dt_next * (1 - trap_next)
    weight = dt * trap + gamma_next
    qk_skip = (q_plain * k_plain).sum(dim=-1) * gamma_next
    scores = torch.einsum("bthn,bshn->bhts", q, k * weight.unsqueeze(-1))
    scores = scores * torch.exp(_segment_sum(adt.transpose(1, 2)))
    y = torch.einsum("bhts,bshd->bthd", scores, x)
    y = y + m.D.float().view(1, 1, H, 1) * x - x * qk_skip.unsqueeze(-1)
    return (y * F.silu(z)).reshape(B, L, m.d_inner)


def mamba3_forward(m, inputs: torch.Tensor) -> torch.Tensor:
    """in_proj, the quadratic mixer, out_proj (python/montlok/rdt/mamba3.py:138-149)."""
    y = mamba3_mixer(m, _linear(inputs.float(), m.in_proj.weight))
    return _linear(y, m.out_proj.weight)

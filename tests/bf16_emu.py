"""What the bf16 kernels compute, restated in torch float64 on the CPU.

The bf16-weight paths round their matrix-core operands to bf16 (round to
nearest even) and accumulate in fp32. This module applies the same roundings
at the same places, with every other operation in float64 and the values the
kernels keep in fp32 rounded to fp32 where the kernels store them:

* linear (bf16 weights): x -> bf16, y = fp32(sum x_bf16 * w).
* MLA forward (mla_window_kernel and the four-launch path, which agree bit
  for bit): x -> bf16; the in_proj columns in fp32; q's rope dims and k_rope
  rotated in fp64 from those fp32 values, rounded to fp32, then bf16; the
  latent LayerNorm'd in fp64, rounded to fp32, then bf16; kv = fp32(latent_bf16
  . W_up^T), k_nope and v rounded to bf16; the causal softmax over key chunks
  of 64 with the running-max rescale of the kernels (max over the raw scores
  scaled once by c = fp32(scale * log2 e) for a positive scale; each
  probability exp2(fp32(s * c - m)) rounded to fp32, summed unrounded, rounded to bf16 for P . V); the output
  O * fp32(1 / l) rounded to fp32, then bf16 for the o_proj.
* attention alone (_C.attention in bf16): the same softmax, fp32 output.

The differences left to the kernels are the fp32 accumulation order of the
matrix cores and the hardware exp2 (about an ulp of fp32 each); where one of
them moves an fp32 value across a bf16 rounding boundary, that one operand
differs by a bf16 ulp.

``round_bf16=False`` turns every rounding off: the chain is then the exact
fp64 forward, which tests/test_bf16_emu.py pins against the oracle's fp32 chain
(so the indexing, RoPE pairing, causal mask and the chunked softmax are pinned
independently of the roundings).
"""

from __future__ import annotations

import math

import numpy as np
import torch

KEY_CHUNK = 64
LOG2E = 1.4426950408889634


class Rounding:
    def __init__(self, on: bool = True):
        self.on = on

    def f32(self, x: torch.Tensor) -> torch.Tensor:
        return x.float().double() if self.on else x

    def bf16(self, x: torch.Tensor) -> torch.Tensor:
        """fp64 -> fp32 -> bf16 (each round to nearest even), as the kernels round a value they hold in fp32."""
        return x.float().bfloat16().double() if self.on else x


def _t(a) -> torch.Tensor:
    return torch.as_tensor(np.asarray(a)).double()


def linear(x, w, bias=None, round_bf16: bool = True):
    """The bf16-weight linear: fp32(bf16(x) . w^T + bias); w holds bf16 values."""
    r = Rounding(round_bf16)
    y = r.bf16(_t(x)) @ _t(w).T
    if bias is not None:
        y = y + _t(bias)
    return r.f32(y).numpy()


def _softmax_pv(s, v_b, visible, scale, r: Rounding):
    """Causal softmax(s * scale) . v over key chunks of 64, as the kernels form it.

    s: [B, H, Lq, Lk] fp32 scores; v_b: [B, H, Lk, hd] bf16 values; visible: [Lq, Lk] bool.
    Returns the fp32 output [B, H, Lq, hd] (before the output rounding)."""
    B, H, Lq, Lk = s.shape
    c = float(np.float32(scale * LOG2E)) if r.on else scale * LOG2E
    m_run = torch.full((B, H, Lq), -math.inf, dtype=torch.float64)
    l_run = torch.zeros((B, H, Lq), dtype=torch.float64)
    o = torch.zeros((B, H, Lq, v_b.shape[-1]), dtype=torch.float64)
    for k0 in range(0, Lk, KEY_CHUNK):
        vis = visible[:, k0:k0 + KEY_CHUNK]
        active = vis.any(-1)  # rows that run this chunk (every causal row with a key in it)
        if not active.any():
            continue
        sc = s[..., k0:k0 + KEY_CHUNK].masked_fill(~vis, -math.inf)
        if c > 0:  # the max over raw scores, scaled once; each exponent one fma
            mx = r.f32(sc.amax(-1) * c)
        else:  # the scores scaled first
            sc = r.f32(sc * c).masked_fill(~vis, -math.inf)
            mx = sc.amax(-1)
        m_new = torch.maximum(m_run, mx)
        m_use = torch.where(m_new == -math.inf, torch.zeros_like(m_new), m_new)
        corr = torch.exp2(r.f32(m_run - m_use))
        e = torch.exp2(r.f32((sc * c if c > 0 else sc) - m_use[..., None]))
        e = r.f32(e).masked_fill(~vis, 0.0)
        a = active[None, None, :]
        l_run = torch.where(a, l_run * corr + e.sum(-1), l_run)
        o = torch.where(a[..., None], o * corr[..., None] + r.bf16(e) @ v_b[..., k0:k0 + KEY_CHUNK, :], o)
        m_run = torch.where(a, m_new, m_run)
    inv = r.f32(1.0 / l_run)
    return r.f32(o * inv[..., None])


def _mask(Lq: int, Lk: int, mask: int) -> torch.Tensor:
    """0: none, 1: causal top-left (key j visible to query i iff j <= i), 2: causal bottom-right."""
    i = torch.arange(Lq)[:, None]
    j = torch.arange(Lk)[None, :]
    if mask == 0:
        return torch.ones(Lq, Lk, dtype=torch.bool)
    return j <= i + (0 if mask == 1 else Lk - Lq)


def attention(q, k, v, mask, scale, round_bf16: bool = True):
    """_C.attention in bf16: q, k, v [B, L, H, hd] rounded to bf16, fp32 output [B, Lq, H, hd]."""
    r = Rounding(round_bf16)
    qb, kb, vb = (r.bf16(_t(a)).permute(0, 2, 1, 3) for a in (q, k, v))
    s = r.f32(qb @ kb.transpose(-1, -2))
    out = _softmax_pv(s, vb, _mask(qb.shape[2], kb.shape[2], mask), scale, r)
    return out.permute(0, 2, 1, 3).numpy()


def _rotate(x, cos, sin, r: Rounding):
    """rotate_half RoPE over the last dim of x [..., L, (heads,) rope] in fp64, rounded to fp32."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return r.f32(torch.cat([x1 * cos[..., :half] - x2 * sin[..., :half],
                            x2 * cos[..., half:] + x1 * sin[..., half:]], -1))


def mla_forward(x, w_q, w_kv_down, w_k_rope, ln_w, ln_b, ln_eps, w_kv_up, w_o, cos, sin, n_heads, head_dim,
                nope_dim, scale, round_bf16: bool = True):
    """The full causal mla_forward with bf16 weights (every query, top-left mask): [B, L, d] fp32."""
    r = Rounding(round_bf16)
    x = _t(x)
    B, L, d = x.shape
    H, hd, nope = n_heads, head_dim, nope_dim
    rope = hd - nope
    xb = r.bf16(x)
    q = r.f32(xb @ _t(w_q).T).reshape(B, L, H, hd)
    latent = r.f32(xb @ _t(w_kv_down).T)
    k_rope = r.f32(xb @ _t(w_k_rope).T)
    cs, sn = _t(cos)[:L], _t(sin)[:L]
    q_rot = _rotate(q[..., nope:], cs[:, None, :], sn[:, None, :], r)
    q_b = r.bf16(torch.cat([q[..., :nope], q_rot], -1))
    kr_b = r.bf16(_rotate(k_rope, cs, sn, r))
    mean = latent.mean(-1, keepdim=True)
    cen = latent - mean
    rstd = 1.0 / torch.sqrt((cen * cen).mean(-1, keepdim=True) + ln_eps)
    ln = cen * rstd * _t(ln_w) + (0.0 if ln_b is None else _t(ln_b))
    kv = r.f32(r.bf16(ln) @ _t(w_kv_up).T).reshape(B, L, H, nope + hd)
    k_b = torch.cat([r.bf16(kv[..., :nope]), kr_b[:, :, None, :].expand(B, L, H, rope)], -1)
    v_b = r.bf16(kv[..., nope:])
    s = r.f32(q_b.permute(0, 2, 1, 3) @ k_b.permute(0, 2, 3, 1))
    att = _softmax_pv(s, v_b.permute(0, 2, 1, 3), _mask(L, L, 1), scale, r)
    att_b = r.bf16(att.permute(0, 2, 1, 3).reshape(B, L, H * hd))
    return r.f32(att_b @ _t(w_o).T).numpy()

"""Pins of the float64 restatement of the bf16 kernels (tests/bf16_emu.py).

With its roundings off the restatement is the exact forward: it must agree
with the oracle's fp32 chain (the indexing, the RoPE pairing, the causal mask
and the chunked softmax against the oracle's one-pass softmax) and with a
direct float64 softmax to rounding error. With them on, the bf16 rounding is
round to nearest even from the fp32 value (ties and the fp64 -> fp32 -> bf16
double rounding checked on known values), and the bf16 linear is the oracle's
product of bf16-rounded inputs.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import bf16_emu as emu
from helpers import rel_err


def _rope_tables(L, rope):
    from montlok.rdt.mla import rope_tables

    return (t.numpy() for t in rope_tables(L, rope))


def test_bf16_rounding_known_values():
    r = emu.Rounding()
    one = 1.0
    vals = torch.tensor([one + 2 ** -8, one + 3 * 2 ** -8, one + 2 ** -8 + 2 ** -30, -(one + 2 ** -7 + 2 ** -9),
                         2.0 ** -130], dtype=torch.float64)
    got = r.bf16(vals).tolist()
    # ties to even; a value just above a tie that fp32 rounds onto it, then the tie rule; a bf16 denormal kept
    assert got == [1.0, one + 2 ** -6, 1.0, -(one + 2 ** -7), 2.0 ** -130]
    assert emu.Rounding(False).bf16(vals).tolist() == vals.tolist()


def test_bf16_linear_is_the_product_of_rounded_inputs(oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((37, 96)).astype(np.float32)
    w = torch.from_numpy(rng.standard_normal((40, 96)) * 0.02).float().bfloat16().float().numpy()
    xb = torch.from_numpy(x).bfloat16().float().numpy()
    assert rel_err(emu.linear(x, w), oracle.linear(xb, w)) <= 1e-7
    assert rel_err(emu.linear(x, w, round_bf16=False), oracle.linear(x, w)) <= 1e-6


@pytest.mark.parametrize("Lq,Lk,mask", [(200, 200, 1), (130, 130, 0), (5, 77, 2), (1, 64, 0), (64, 64, 1)])
def test_chunked_softmax_is_the_softmax(Lq, Lk, mask):
    """Without roundings the 64-key chunks with the running-max rescale equal one softmax over all keys."""
    g = torch.Generator().manual_seed(Lq + Lk)
    q, k, v = (torch.randn(2, n, 3, 16, generator=g, dtype=torch.float64) for n in (Lq, Lk, Lk))
    scale = 0.3
    got = emu.attention(q.numpy(), k.numpy(), v.numpy(), mask, scale, round_bf16=False)
    s = torch.einsum("bqhd,bkhd->bhqk", q, k) * scale
    s = s.masked_fill(~emu._mask(Lq, Lk, mask), -math.inf)
    expect = torch.einsum("bhqk,bkhd->bqhd", torch.softmax(s, -1), v)
    assert np.abs(got - expect.numpy()).max() <= 1e-12


def test_attention_unrounded_vs_oracle(oracle):
    rng = np.random.default_rng(8)
    q, k, v = (rng.standard_normal((2, 150, 2, 32)).astype(np.float32) for _ in range(3))
    for mask in (0, 1):
        got = emu.attention(q, k, v, mask, 32 ** -0.5, round_bf16=False)
        assert rel_err(got, oracle.sdpa(q, k, v, mask, 32 ** -0.5)) <= 2e-6


def _mla_case(rng, B, L, H, hd, nope, kvr, std):
    d, rope = H * hd, hd - nope
    x = rng.standard_normal((B, L, d)).astype(np.float32)
    w = {n: (rng.standard_normal(s) * std).astype(np.float32) for n, s in
         (("q", (d, d)), ("kv_down", (kvr, d)), ("k_rope", (rope, d)), ("kv_up", (H * (nope + hd), kvr)),
          ("o", (d, d)))}
    ln_w = (1 + 0.1 * rng.standard_normal(kvr)).astype(np.float32)
    ln_b = (0.1 * rng.standard_normal(kvr)).astype(np.float32)
    return x, w, ln_w, ln_b


def _oracle_chain(oracle, x, w, ln_w, ln_b, cos, sin, H, hd, nope, scale):
    B, L, d = x.shape
    q = oracle.linear(x, w["q"]).reshape(B, L, H, hd)
    lat = oracle.linear(x, w["kv_down"])
    kr = oracle.linear(x, w["k_rope"])
    kv = oracle.linear(oracle.layer_norm(lat, ln_w, ln_b, 1e-5), w["kv_up"]).reshape(B, L, H, nope + hd)
    q, k = oracle.mla_rope(q, kv, kr, cos, sin, nope)
    att = oracle.sdpa(q, k, np.ascontiguousarray(kv[..., nope:]), 1, scale)
    return oracle.linear(att.reshape(B, L, d), w["o"])


@pytest.mark.parametrize("B,L,H,hd,nope", [(2, 128, 8, 32, 16), (1, 200, 4, 64, 32)])
def test_mla_unrounded_vs_oracle_chain(oracle, B, L, H, hd, nope):
    rng = np.random.default_rng(L)
    x, w, ln_w, ln_b = _mla_case(rng, B, L, H, hd, nope, 64, 0.08)
    cos, sin = _rope_tables(L, hd - nope)
    scale = hd ** -0.5
    got = emu.mla_forward(x, w["q"], w["kv_down"], w["k_rope"], ln_w, ln_b, 1e-5, w["kv_up"], w["o"], cos, sin, H, hd,
                          nope, scale, round_bf16=False)
    expect = _oracle_chain(oracle, x, w, ln_w, ln_b, cos, sin, H, hd, nope, scale)
    assert rel_err(got, expect) <= 2e-6
    # The roundings move the result by bf16's precision, no more: within the 2e-2 contract, above fp32 noise.
    rounded = emu.mla_forward(x, w["q"], w["kv_down"], w["k_rope"], ln_w, ln_b, 1e-5, w["kv_up"], w["o"], cos, sin,
                              H, hd, nope, scale)
    assert 1e-4 <= rel_err(rounded, expect) <= 2e-2

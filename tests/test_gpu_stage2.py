"""GPU parity of stage2_tail_forward (montlok.cpp:1217-1359), the recurrent
stage-2 mHC tail: `depth` applications of one layer (attention residual over
MLA, FFN residual over a SwiGLU MLP) from a broadcast backbone to the
collapsed last token. The packed op is compared with the same chain of
oracle ops: 1e-5 normwise for fp32 weights, 2e-2 for bf16 weights."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import BF16_TOL, assert_close
from test_gpu_modules import _mla_oracle, _np

pytestmark = pytest.mark.gpu


def _layer(d_model: int, ffn_hidden: int, n_streams: int, seed: int):
    from montlok.rdt import MLAHIP, ManifoldHyperConnectionHIP, RMSNormHIP, SwiGLUHIP

    torch.manual_seed(seed)
    cfg = SimpleNamespace(d_model=d_model, n_heads=8, head_dim=32, nope_head_dim=16, rope_head_dim=16,
                          kv_lora_rank=64, q_lora_rank=0, rope_theta=10000.0)
    layer = SimpleNamespace(attn_hc=ManifoldHyperConnectionHIP(d_model, n_streams),
                            ffn_hc=ManifoldHyperConnectionHIP(d_model, n_streams),
                            attn_norm=RMSNormHIP(d_model), ffn_norm=RMSNormHIP(d_model),
                            attn=MLAHIP(cfg).eval(), ffn=SwiGLUHIP(d_model, ffn_hidden, bias=True))
    with torch.no_grad():
        for hc in (layer.attn_hc, layer.ffn_hc):
            for a in (hc.pre_alpha, hc.post_alpha, hc.res_alpha):
                a.fill_(0.7)
            for p in (hc.pre_proj.weight, hc.post_proj.weight, hc.res_proj.weight):
                p.normal_(0.0, d_model ** -0.5)
            hc.res_bias.normal_()
        for nm in (layer.attn_norm, layer.ffn_norm):
            nm.weight.normal_(1.0, 0.1)
        layer.attn.kv_norm.weight.normal_(1.0, 0.1)
        layer.attn.kv_norm.bias.normal_(0.0, 0.1)
        layer.ffn.w_in.bias.normal_(0.0, 0.1)
        layer.ffn.w_down.bias.normal_(0.0, 0.1)
    return layer


def _round_bf16(layer):
    a, f = layer.attn, layer.ffn
    with torch.no_grad():
        for lin in (a.q_proj, a.kv_down, a.kv_up, a.k_rope_proj, a.o_proj, f.w_in, f.w_down):
            lin.weight.normal_(0.0, 0.02)
            lin.weight.copy_(lin.weight.bfloat16().float())


def _packs(layer, L: int, dev, bf16: bool):
    """The tensor packs of model.py:160-232, on the device (bf16 projection weights when asked)."""
    a, f = layer.attn, layer.ffn
    w = (lambda t: t.detach().to(dev, torch.bfloat16)) if bf16 else (lambda t: t.detach().to(dev))
    empty = torch.empty(0, device=dev)

    def hc_pack(hc):
        return (hc.dyn_norm.weight.detach().to(dev), hc._projection_block().to(dev), hc.pre_bias.detach().to(dev),
                hc.post_bias.detach().to(dev), hc.res_bias.detach().to(dev), hc.pre_alpha.detach().to(dev),
                hc.post_alpha.detach().to(dev), hc.res_alpha.detach().to(dev))

    cos, sin = a._rope_tables(L, 0, dev)
    mla = (w(a._in_proj_weight(True)), w(a._in_proj_weight(False)), w(a.q_proj.weight),
           a.kv_norm.weight.detach().to(dev), a.kv_norm.bias.detach().to(dev) if a.kv_norm.bias is not None else empty,
           w(a.kv_up.weight), w(a.o_proj.weight), cos, sin)
    ffn = (w(f.w_in.weight), f.w_in.bias.detach().to(dev), w(f.w_down.weight), f.w_down.bias.detach().to(dev))
    return hc_pack(layer.attn_hc), mla, hc_pack(layer.ffn_hc), ffn


def _oracle_tail(oracle, layer, backbone: np.ndarray, depth: int) -> np.ndarray:
    from montlok.rdt.mla import rope_tables

    B, L, _ = backbone.shape
    n = layer.attn_hc.n_streams
    cos, sin = (t.numpy() for t in rope_tables(L, layer.attn.rope_dim))

    def prepare(hc, norm, streams, n_streams):
        return oracle.mhc_prepare(streams, _np(hc.dyn_norm.weight), hc.dyn_norm.eps,
                                  hc._projection_block().cpu().numpy(), _np(hc.pre_bias), _np(hc.post_bias),
                                  _np(hc.res_bias), float(hc.pre_alpha.detach()), float(hc.post_alpha.detach()),
                                  float(hc.res_alpha.detach()),
                                  hc.sinkhorn_iters, n_streams, _np(norm.weight), norm.eps)

    def ffn(x):
        f = layer.ffn
        bias = (lambda b: None if b is None else _np(b))  # noqa: E731
        h = oracle.linear(x, _np(f.w_in.weight), bias(f.w_in.bias))
        return oracle.linear(oracle.swiglu(h), _np(f.w_down.weight), bias(f.w_down.bias))

    agg, _, post, res = prepare(layer.attn_hc, layer.attn_norm, backbone, n)
    streams = backbone
    for step in range(depth):
        if step + 1 == depth:
            att = _mla_oracle(oracle, layer.attn, agg, 1, 0, cos, sin)
            written = oracle.mhc_combine(np.ascontiguousarray(streams[:, L - 1:]), np.ascontiguousarray(res[:, L - 1:]),
                                         np.ascontiguousarray(post[:, L - 1:]), att)
            f_agg, _, f_post, f_res = prepare(layer.ffn_hc, layer.ffn_norm, written, 0)
            return oracle.mhc_combine(written, f_res, f_post, ffn(f_agg), collapse=True, materialize=False)
        att = _mla_oracle(oracle, layer.attn, agg, L, 1, cos, sin)
        streams = oracle.mhc_combine(streams, res, post, att)
        f_agg, _, f_post, f_res = prepare(layer.ffn_hc, layer.ffn_norm, streams, 0)
        streams = oracle.mhc_combine(streams, f_res, f_post, ffn(f_agg))
        agg, _, post, res = prepare(layer.attn_hc, layer.attn_norm, streams, 0)
    raise AssertionError("unreachable")


def _run(layer, backbone: torch.Tensor, depth: int, bf16: bool):
    from montlok import _C

    dev = backbone.device
    attn_hc, mla, ffn_hc, ffn = _packs(layer, backbone.shape[1], dev, bf16)
    a = layer.attn
    return _C.stage2_tail_forward(backbone, depth, layer.attn_hc.n_streams, attn_hc, layer.attn_hc.dyn_norm.eps,
                                  layer.attn_hc.sinkhorn_iters, layer.attn_norm.weight.detach().to(dev),
                                  layer.attn_norm.eps, mla, a.kv_norm.eps, a.n_heads, a.head_dim, a.nope_dim,
                                  a.kv_lora_rank, a.scale, ffn_hc, layer.ffn_hc.dyn_norm.eps,
                                  layer.ffn_hc.sinkhorn_iters, layer.ffn_norm.weight.detach().to(dev),
                                  layer.ffn_norm.eps, ffn)


@pytest.mark.parametrize("depth,B,L", [(1, 2, 24), (2, 2, 24), (3, 3, 40)])
def test_stage2_tail_vs_oracle(dev, oracle, depth, B, L):
    layer = _layer(256, 384, 4, seed=depth)
    backbone = torch.randn(B, L, 256, generator=torch.Generator().manual_seed(10 + depth))
    with torch.no_grad():
        got = _run(layer, backbone.to(dev), depth, bf16=False)
    assert tuple(got.shape) == (B, 1, 256)
    assert_close(got, _oracle_tail(oracle, layer, backbone.numpy(), depth), tol=1e-5, name=f"stage2 depth {depth}")


def test_stage2_tail_bf16_weights(dev, oracle):
    layer = _layer(256, 384, 4, seed=11)
    _round_bf16(layer)
    backbone = torch.randn(2, 32, 256, generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        got = _run(layer, backbone.to(dev), 2, bf16=True)
    assert_close(got, _oracle_tail(oracle, layer, backbone.numpy(), 2), tol=BF16_TOL, name="stage2 bf16")


@pytest.mark.parametrize("n_streams", [4, 3])
def test_stage2_buffer_variants_same_values(dev, monkeypatch, n_streams):
    """MONTLOK_STAGE2_INPLACE and MONTLOK_STAGE2_REUSE_COEFF (montlok.cpp:1291-1295) change only where the
    streams and coefficients live: all four combinations give the same bits, and the in-place,
    coefficient-reusing default holds less device memory at its peak than neither."""
    layer = _layer(256, 384, n_streams, seed=21)
    backbone = torch.randn(4, 64, 256, generator=torch.Generator().manual_seed(4)).to(dev)
    results, peaks = {}, {}
    for inplace in ("1", "0"):
        for reuse in ("1", "0"):
            monkeypatch.setenv("MONTLOK_STAGE2_INPLACE", inplace)
            monkeypatch.setenv("MONTLOK_STAGE2_REUSE_COEFF", reuse)
            with torch.no_grad():
                _run(layer, backbone, 3, bf16=False)  # warm the caches and packs
                torch.cuda.synchronize()
                torch.cuda.reset_peak_memory_stats()
                base = torch.cuda.memory_allocated()
                results[(inplace, reuse)] = _run(layer, backbone, 3, bf16=False)
                torch.cuda.synchronize()
                peaks[(inplace, reuse)] = torch.cuda.max_memory_allocated() - base
    ref = results[("0", "0")]
    for key, got in results.items():
        assert torch.equal(got, ref), f"INPLACE={key[0]} REUSE_COEFF={key[1]}"
    assert peaks[("1", "1")] < peaks[("0", "0")], peaks

"""GPU parity of the drop-in modules (montlok.rdt) against the oracle applied
to the same parameters: Mamba-3 forward and streaming step, the mHC residual
(forward, forward_tail, expand/collapse), MLA (full causal, one trailing query,
several trailing queries) and the per-token layers. Gates: 1e-5 normwise for
fp32 weights, 2e-2 for bf16 weights."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import BF16_TOL, assert_bitwise, assert_close

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


def _mamba_oracle(oracle, m, x):
    p = dict(b=_np(m.B_bias), c=_np(m.C_bias), bw=_np(m.B_norm.weight), cw=_np(m.C_norm.weight),
             dt=_np(m.dt_bias), skip=_np(m.D))
    projected = oracle.linear(x, _np(m.in_proj.weight))
    y = oracle.mamba3_siso_forward(projected, m.d_state, m.num_bc_heads, m.nheads, m.headdim, m.num_rope_angles,
                                   p["b"], p["c"], p["bw"], p["cw"], 1e-5, 1e-5, p["dt"], p["skip"], m.A_floor)
    return oracle.linear(y, _np(m.out_proj.weight))


def test_mamba3_module_forward_and_step(dev, oracle):
    from montlok.rdt import Mamba3HIP

    torch.manual_seed(0)
    m = Mamba3HIP(64, d_state=16, expand=2, headdim=32).to(dev).eval()
    with torch.no_grad():
        m.B_bias.add_(0.3 * torch.randn_like(m.B_bias))
        m.C_bias.add_(0.3 * torch.randn_like(m.C_bias))
    x = torch.randn(3, 20, 64)
    with torch.no_grad():
        out = m(x.to(dev))
        assert_close(out, _mamba_oracle(oracle, m, x.numpy()), name="Mamba3HIP.forward")
        # T steps from a zero state reproduce the forward over those T tokens.
        state = m.new_state(3)
        steps = torch.stack([m.step(x[:, t].to(dev), state) for t in range(20)], dim=1)
    assert_close(steps, out, tol=1e-6, name="step x T vs forward")


def _mhc_oracle(oracle, h, streams, fn):
    w64 = h._projection_block().cpu().numpy()
    agg, pre, post, res = oracle.mhc_prepare(streams, _np(h.dyn_norm.weight), h.dyn_norm.eps, w64, _np(h.pre_bias),
                                             _np(h.post_bias), _np(h.res_bias), float(h.pre_alpha),
                                             float(h.post_alpha), float(h.res_alpha), h.sinkhorn_iters)
    return oracle.mhc_combine(streams, res, post, fn(agg)), agg


def test_mhc_module_forward_tail_and_collapse(dev, oracle):
    from montlok.rdt import ManifoldHyperConnectionHIP

    torch.manual_seed(1)
    h = ManifoldHyperConnectionHIP(128, n_streams=4).to(dev)
    with torch.no_grad():
        for a in (h.pre_alpha, h.post_alpha, h.res_alpha):
            a.fill_(0.7)
        for p in (h.pre_proj.weight, h.post_proj.weight, h.res_proj.weight):
            p.normal_(0.0, 128 ** -0.5)
        h.res_bias.normal_()
    x = torch.randn(2, 16, 128)
    streams = h.expand(x.to(dev)).contiguous()
    s_np = streams.cpu().numpy()
    with torch.no_grad():
        out = h(streams, lambda agg: agg * 0.5)
        expect, agg = _mhc_oracle(oracle, h, s_np, lambda a: a * 0.5)
        assert_close(out, expect, name="mHC forward")
        tail = h.forward_tail(streams, lambda a: a[:, -3:] * 0.5, n_last=3)
        assert_close(tail, expect[:, -3:], name="mHC forward_tail")
        assert_close(h.collapse(out), expect.mean(axis=-2), name="collapse")


def _mla_cfg(q_lora=0):
    return SimpleNamespace(d_model=256, n_heads=8, head_dim=32, nope_head_dim=16, rope_head_dim=16, kv_lora_rank=64,
                           q_lora_rank=q_lora, rope_theta=10000.0)


def _mla_oracle(oracle, m, x, n_last, mask, cos, sin):
    B, L, d = x.shape
    H, hd, nope, kvr = m.n_heads, m.head_dim, m.nope_dim, m.kv_lora_rank
    kv_lat = oracle.linear(x, _np(m.kv_down.weight))
    k_rope = oracle.linear(x, _np(m.k_rope_proj.weight))
    q = oracle.linear(x[:, L - n_last:], _np(m.q_proj.weight)).reshape(B, n_last, H, hd)
    kv = oracle.linear(oracle.layer_norm(kv_lat, _np(m.kv_norm.weight), _np(m.kv_norm.bias), 1e-5),
                       _np(m.kv_up.weight)).reshape(B, L, H, nope + hd)
    q, k = oracle.mla_rope(q, kv, k_rope, cos, sin, nope)
    att = oracle.sdpa(q, k, np.ascontiguousarray(kv[..., nope:]), mask, m.scale)
    return oracle.linear(att.reshape(B, n_last, d), _np(m.o_proj.weight))


@pytest.mark.parametrize("bf16", [False, True])
def test_mla_module(dev, oracle, bf16):
    from montlok.rdt import MLAHIP
    from montlok.rdt.mla import rope_tables

    torch.manual_seed(2)
    m = MLAHIP(_mla_cfg()).eval()
    with torch.no_grad():
        m.kv_norm.weight.normal_(1.0, 0.1)
        m.kv_norm.bias.normal_(0.0, 0.1)
        if bf16:
            for lin in (m.q_proj, m.kv_down, m.kv_up, m.k_rope_proj, m.o_proj):
                lin.weight.normal_(0.0, 0.02)
                lin.weight.copy_(lin.weight.bfloat16().float())
    ref_m = m
    m = m.to(dev)
    if bf16:
        for lin in (m.q_proj, m.kv_down, m.kv_up, m.k_rope_proj, m.o_proj):
            lin.to(torch.bfloat16)
    x = torch.randn(4, 40, 256)
    cos, sin = (t.numpy() for t in rope_tables(40, 16))
    tol = BF16_TOL if bf16 else 1e-5
    with torch.no_grad():
        full = m(x.to(dev))
        assert_close(full, _mla_oracle(oracle, ref_m, x.numpy(), 40, 1, cos, sin), tol=tol, name="MLA forward")
        last = m.forward_last(x.to(dev), 1)
        assert_close(last, _mla_oracle(oracle, ref_m, x.numpy(), 1, 0, cos, sin), tol=tol, name="MLA forward_last(1)")
        last3 = m.forward_last(x.to(dev), 3)
        assert_close(last3, _mla_oracle(oracle, ref_m, x.numpy(), 3, 2, cos, sin), tol=tol,
                     name="MLA forward_last(3), bottom-right mask")
        # The trailing rows of the full causal forward are the same attention as forward_last.
        assert_close(last3, full[:, -3:], tol=tol, name="forward_last(3) vs full[-3:]")


def test_layer_modules(dev, oracle):
    from montlok.rdt import GroupedRMSNormCPU, LayerNormCPU, RMSNormCPU, SwiGLUCPU

    torch.manual_seed(3)
    x = torch.randn(5, 7, 64)
    xd = x.to(dev)
    with torch.no_grad():
        g = GroupedRMSNormCPU(64, 8).to(dev)
        g.weight.normal_(1.0, 0.1)
        assert_bitwise(g(xd), oracle.rms_norm(x.numpy(), _np(g.weight), 1e-5, 8), "GroupedRMSNorm")
        r = RMSNormCPU(64).to(dev)
        assert_bitwise(r(xd), oracle.rms_norm(x.numpy(), _np(r.weight), 1e-5, 1), "RMSNorm")
        ln = LayerNormCPU(64).to(dev)
        ln.bias.normal_(0.0, 0.1)
        assert_bitwise(ln(xd), oracle.layer_norm(x.numpy(), _np(ln.weight), _np(ln.bias), 1e-5), "LayerNorm")
        s = SwiGLUCPU(64, 96, bias=True).to(dev)
        expect = oracle.linear(oracle.swiglu(oracle.linear(x.numpy(), _np(s.w_in.weight), _np(s.w_in.bias))),
                               _np(s.w_down.weight), _np(s.w_down.bias))
        assert_close(s(xd), expect, name="SwiGLU")

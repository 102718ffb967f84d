"""The upstream PyTorch forwards the modules run when a switch turns the kernels off (MONTLOK_CPP=0,
MONTLOK_CPP_MHC=0, MONTLOK_CPP_LAYERS=0; README.md:268-271 of the reference), on the CPU against the
oracle: these are the tensor programs of the upstream formulas, so they agree with the kernels' arithmetic
to the reference's own tolerance for a PyTorch-vs-kernel pair, 2e-5 (1 + max|y|)
(tests/rdt/test_rdt_kernels.py:126-128), not bit for bit."""

from __future__ import annotations

import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import to_np


def _ref_tol(actual, expected, tol=2e-5, name=""):
    a, e = to_np(actual).astype(np.float64), np.asarray(to_np(expected), dtype=np.float64)
    assert a.shape == e.shape and np.isfinite(a).all(), name
    diff = np.abs(a - e).max()
    assert diff <= tol * (1.0 + np.abs(e).max()), f"{name}: max|diff| {diff:.3e}"
    return diff


@pytest.fixture
def torch_env(monkeypatch):
    monkeypatch.setenv("MONTLOK_CPP", "0")
    return monkeypatch


def _np(t):
    return t.detach().float().numpy()


def test_layers(oracle, torch_env):
    from montlok.rdt import GroupedRMSNormHIP, LayerNormHIP, RMSNormHIP, SwiGLUHIP

    torch.manual_seed(1)
    x = torch.randn(4, 9, 64)
    with torch.no_grad():
        n = RMSNormHIP(64)
        n.weight.normal_(1.0, 0.1)
        _ref_tol(n(x), oracle.rms_norm(x.numpy(), _np(n.weight), 1e-5, 1), name="RMSNorm")
        g = GroupedRMSNormHIP(64, num_groups=8)
        g.weight.normal_(1.0, 0.1)
        _ref_tol(g(x), oracle.rms_norm(x.numpy(), _np(g.weight), 1e-5, 8), name="GroupedRMSNorm")
        ln = LayerNormHIP(64)
        ln.weight.normal_(1.0, 0.1)
        ln.bias.normal_(0.0, 0.1)
        _ref_tol(ln(x), oracle.layer_norm(x.numpy(), _np(ln.weight), _np(ln.bias), 1e-5), name="LayerNorm")
        f = SwiGLUHIP(64, 96, bias=True)
        expect = oracle.linear(oracle.swiglu(oracle.linear(x.numpy(), _np(f.w_in.weight), _np(f.w_in.bias))),
                               _np(f.w_down.weight), _np(f.w_down.bias))
        _ref_tol(f(x), expect, name="SwiGLU")


@pytest.mark.parametrize("d_model,d_state,headdim,ngroups,L", [(64, 16, 32, 1, 40), (48, 14, 8, 2, 23)])
def test_mamba3(oracle, torch_env, d_model, d_state, headdim, ngroups, L):
    from montlok.rdt import Mamba3HIP

    torch.manual_seed(3)
    m = Mamba3HIP(d_model, d_state=d_state, expand=2, headdim=headdim, ngroups=ngroups).eval()
    with torch.no_grad():
        m.B_bias.add_(0.3 * torch.randn_like(m.B_bias))
        m.C_bias.add_(0.3 * torch.randn_like(m.C_bias))
        m.D.add_(0.5 * torch.randn_like(m.D))
        x = torch.randn(2, L, d_model)
        got = m(x)
    p = dict(b=_np(m.B_bias), c=_np(m.C_bias), bw=_np(m.B_norm.weight), cw=_np(m.C_norm.weight),
             dt=_np(m.dt_bias), skip=_np(m.D))
    projected = oracle.linear(x.numpy(), _np(m.in_proj.weight))
    y = oracle.mamba3_siso_forward(projected, m.d_state, m.num_bc_heads, m.nheads, m.headdim, m.num_rope_angles,
                                   p["b"], p["c"], p["bw"], p["cw"], 1e-5, 1e-5, p["dt"], p["skip"], m.A_floor)
    _ref_tol(got, oracle.linear(y, _np(m.out_proj.weight)), name="Mamba-3 quadratic form")


def test_mhc(oracle, torch_env):
    from montlok.rdt import ManifoldHyperConnectionHIP

    torch.manual_seed(4)
    h = ManifoldHyperConnectionHIP(64, n_streams=4)
    with torch.no_grad():
        for a in (h.pre_alpha, h.post_alpha, h.res_alpha):
            a.fill_(0.7)
        for p in (h.pre_proj.weight, h.post_proj.weight, h.res_proj.weight):
            p.normal_(0.0, 64 ** -0.5)
        h.res_bias.normal_()
        streams = torch.randn(2, 11, 4, 64)
        out = h(streams, lambda agg: torch.tanh(agg))
        tail = h.forward_tail(streams, lambda agg: torch.tanh(agg[:, -2:]), n_last=2)
    s = streams.numpy()
    agg, pre, post, res = oracle.mhc_prepare(s, _np(h.dyn_norm.weight), h.dyn_norm.eps,
                                             h._projection_block().numpy(), _np(h.pre_bias), _np(h.post_bias),
                                             _np(h.res_bias), 0.7, 0.7, 0.7, h.sinkhorn_iters)
    expect = oracle.mhc_combine(s, res, post, np.tanh(agg))
    _ref_tol(out, expect, name="mHC forward (log-space Sinkhorn)")
    _ref_tol(tail, expect[:, -2:], name="mHC forward_tail")
    # Unconstrained residual (softplus), which only this path computes: rows are not normalised.
    h.constrain = False
    with torch.no_grad():
        free = h(streams, lambda agg: agg * 0.0)
    assert not torch.allclose(free, out)


@pytest.mark.parametrize("n_last", [24, 1, 3])
def test_mla(oracle, torch_env, n_last):
    from montlok.rdt import MLAHIP
    from montlok.rdt.mla import rope_tables

    torch.manual_seed(5)
    cfg = SimpleNamespace(d_model=64, n_heads=2, head_dim=32, nope_head_dim=16, rope_head_dim=16, kv_lora_rank=32,
                          q_lora_rank=0, rope_theta=10000.0)
    m = MLAHIP(cfg).eval()
    with torch.no_grad():
        m.kv_norm.weight.normal_(1.0, 0.1)
        m.kv_norm.bias.normal_(0.0, 0.1)
        x = torch.randn(2, 24, 64)
        got = m(x) if n_last == 24 else m.forward_last(x, n_last)
    B, L, d = x.shape
    H, hd, nope = 2, 32, 16
    cos, sin = (t.numpy() for t in rope_tables(L, 16))
    xn = x.numpy()
    kv = oracle.linear(oracle.layer_norm(oracle.linear(xn, _np(m.kv_down.weight)), _np(m.kv_norm.weight),
                                         _np(m.kv_norm.bias), 1e-5), _np(m.kv_up.weight)).reshape(B, L, H, nope + hd)
    q = oracle.linear(xn[:, L - n_last:], _np(m.q_proj.weight)).reshape(B, n_last, H, hd)
    q, k = oracle.mla_rope(q, kv, oracle.linear(xn, _np(m.k_rope_proj.weight)), cos, sin, nope)
    mask = 1 if n_last == L else (0 if n_last == 1 else 2)
    att = oracle.sdpa(q, k, np.ascontiguousarray(kv[..., nope:]), mask, 1 / math.sqrt(hd))
    _ref_tol(got, oracle.linear(att.reshape(B, n_last, d), _np(m.o_proj.weight)), name=f"MLA n_last={n_last}")


def test_model_runs_the_module_chain(torch_env):
    """With MONTLOK_CPP=0 the model runs on the CPU through the modules' upstream forwards (the reference's
    stock path), finite and with the shapes of the kernel path."""
    from montlok.rdt import RDT4QuantHIP
    from test_modules import _tiny_model_config

    torch.manual_seed(0)
    m = RDT4QuantHIP(7, _tiny_model_config()).eval()
    with torch.no_grad():
        q, rms = m(torch.randn(2, 12, 7), 2)
    assert q.shape[-1] == 3 and torch.isfinite(q).all() and torch.isfinite(rms)

"""GPU parity of the hybrid stack (feature projection, 4 mHC residual layers
alternating Mamba-3 and MLA, collapse) against the same chain of oracle ops:
fp32 weights within 1e-5, bf16 weights within 2e-2 (normwise); with bf16
weights each wrapped layer also against the chain with the bf16 kernels'
roundings (tests/bf16_emu.py) on the layer's own GPU input.

Two geometries: a small one (d_model 64, d_state 16, 2 MLA heads of 32,
kv rank 32, 2 x 32 tokens), and the full stack's own (d_model 256, d_state 64,
Mamba-3 8 heads of 64, MLA 4 heads of 64 with RoPE 32 and kv rank 64, n = 4
streams, 20 Sinkhorn iterations, 40 features; reference/Model/two_stage.py
:98-116, 402-409 with reference/config.json:27-46) on 2 windows x 256 tokens,
which takes the same fused kernels as the 1024-window workload (the MLA
attend form with head_dim 64 / nope 32, the d-256 combine+prepare)."""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

import bf16_emu as emu
from helpers import BF16_TOL, assert_close, assert_emulated, rel_err, row_errors
from test_gpu_modules import _mla_oracle, _np

pytestmark = pytest.mark.gpu


def _randomise(stack, bf16: bool):
    torch.manual_seed(5)
    with torch.no_grad():
        for hc in stack.hcs:
            for a in (hc.pre_alpha, hc.post_alpha, hc.res_alpha):
                a.fill_(0.7)
            for p in (hc.pre_proj.weight, hc.post_proj.weight, hc.res_proj.weight):
                p.normal_(0.0, stack.d_model ** -0.5)
            hc.res_bias.normal_()
        for n in stack.norms:
            n.weight.normal_(1.0, 0.1)
        for m in stack.mixers:
            if hasattr(m, "B_bias"):
                m.B_bias.add_(0.3 * torch.randn_like(m.B_bias))
        if bf16:
            for w in stack.linear_weights():
                w.normal_(0.0, 0.02)
                w.copy_(w.bfloat16().float())


def _mixer_chain(oracle, m, x, cos, sin, bf16_emulation: bool):
    """One wrapped layer (Mamba-3 or MLA) on x as oracle ops; with bf16_emulation its GEMMs and the MLA are
    the float64 restatement of the bf16 kernels (tests/bf16_emu.py) and the Mamba-3 scan stays the oracle's."""
    lin = emu.linear if bf16_emulation else oracle.linear
    if hasattr(m, "B_bias"):
        p = dict(b=_np(m.B_bias), c=_np(m.C_bias), bw=_np(m.B_norm.weight), cw=_np(m.C_norm.weight),
                 dt=_np(m.dt_bias), skip=_np(m.D))
        y = oracle.mamba3_siso_forward(lin(x, _np(m.in_proj.weight)), m.d_state, m.num_bc_heads, m.nheads, m.headdim,
                                       m.num_rope_angles, p["b"], p["c"], p["bw"], p["cw"], 1e-5, 1e-5, p["dt"],
                                       p["skip"], m.A_floor)
        return lin(y, _np(m.out_proj.weight))
    if not bf16_emulation:
        return _mla_oracle(oracle, m, x, x.shape[1], 1, cos, sin)
    return emu.mla_forward(x, _np(m.q_proj.weight), _np(m.kv_down.weight), _np(m.k_rope_proj.weight),
                           _np(m.kv_norm.weight), _np(m.kv_norm.bias), m.kv_norm.eps, _np(m.kv_up.weight),
                           _np(m.o_proj.weight), cos, sin, m.n_heads, m.head_dim, m.nope_dim, m.scale)


def _rope(stack, L):
    from montlok.rdt.mla import rope_tables

    return (t.numpy() for t in rope_tables(L, stack.mixers[1].rope_dim))


def _oracle_stack(oracle, stack, feats, bf16_emulation: bool = False):
    """The stack as a chain of oracle ops (with bf16_emulation: the bf16 kernels' GEMMs and MLA restated)."""
    B, L, _ = feats.shape
    cos, sin = _rope(stack, L)
    lin = emu.linear if bf16_emulation else oracle.linear
    h = lin(feats, _np(stack.feature_proj.weight), _np(stack.feature_proj.bias))

    def mixer(i, x):
        return _mixer_chain(oracle, stack.mixers[i], x, cos, sin, bf16_emulation)

    def prepare(i, streams, n_streams):
        hc = stack.hcs[i]
        return oracle.mhc_prepare(streams, _np(hc.dyn_norm.weight), hc.dyn_norm.eps,
                                  hc._projection_block().cpu().numpy(), _np(hc.pre_bias), _np(hc.post_bias),
                                  _np(hc.res_bias), float(hc.pre_alpha.detach()), float(hc.post_alpha.detach()),
                                  float(hc.res_alpha.detach()),
                                  hc.sinkhorn_iters, n_streams, _np(stack.norms[i].weight), stack.norms[i].eps)

    agg, pre, post, res = prepare(0, h, stack.n_streams)
    out = mixer(0, agg)
    streams = h
    for i in range(1, len(stack.hcs)):
        streams = oracle.mhc_combine(streams, res, post, out)
        agg, pre, post, res = prepare(i, streams, 0)
        out = mixer(i, agg)
    return oracle.mhc_combine(streams, res, post, out, collapse=True, materialize=False)


GEOMETRIES = {
    "small": (dict(d_model=64, d_state=16, mamba_headdim=32, n_heads=2, head_dim=32, rope_head_dim=16,
                   kv_lora_rank=32), 32),
    "stack": (dict(d_model=256, d_state=64, mamba_headdim=64, n_heads=4, head_dim=64, rope_head_dim=32,
                   kv_lora_rank=64), 256),
}


@pytest.mark.parametrize("geometry", sorted(GEOMETRIES))
@pytest.mark.parametrize("bf16", [False, True])
def test_hybrid_stack(dev, oracle, bf16, geometry):
    from montlok.rdt.stack import HybridStackHIP

    kwargs, L = GEOMETRIES[geometry]
    stack = HybridStackHIP(40, n_layers=4, n_streams=4, **kwargs).eval()
    _randomise(stack, bf16)
    feats = np.clip(np.random.default_rng(6).standard_normal((2, L, 40)), -8, 8).astype(np.float32)
    expect = _oracle_stack(oracle, stack, feats)
    stack_cpu = copy.deepcopy(stack)
    stack = stack.to(dev)
    if bf16:
        for w in stack.linear_weights():
            w.data = w.data.bfloat16()
    seen = []
    hooks = [mx.register_forward_hook(lambda mod, inp, out: seen.append((inp[0].cpu().numpy(), out.cpu().numpy())))
             for mx in stack.mixers]
    with torch.no_grad():
        out = stack(torch.from_numpy(feats).to(dev))
    for hk in hooks:
        hk.remove()
    assert out.shape == (2, L, kwargs["d_model"])
    err = assert_close(out, expect, tol=BF16_TOL if bf16 else 1e-5, name=f"hybrid stack {geometry} bf16={bf16}")
    if bf16:
        # What the bf16 kernels compute, layer by layer: each wrapped layer's output against the float64
        # restatement of its roundings applied to the layer's own GPU input. End to end, the bf16 roundings
        # of operands that the layers before moved by an fp32 ulp compound, so the whole chain is printed.
        cos, sin = _rope(stack_cpu, L)
        assert len(seen) == len(stack_cpu.mixers)
        for i, (x_in, y_out) in enumerate(seen):
            want = _mixer_chain(oracle, stack_cpu.mixers[i], x_in, cos, sin, True)
            e, m = assert_emulated(y_out, want, name=f"hybrid stack {geometry} layer {i} vs the bf16 emulation")
            print(f"hybrid stack {geometry} layer {i} ({type(stack_cpu.mixers[i]).__name__}): vs the bf16 "
                  f"emulation {e:.2e} (median row {m:.1e}), vs its fp32 chain "
                  f"{rel_err(y_out, _mixer_chain(oracle, stack_cpu.mixers[i], x_in, cos, sin, False)):.2e}")
        emulated = _oracle_stack(oracle, stack_cpu, feats, bf16_emulation=True)
        print(f"hybrid stack {geometry} bf16 end to end: vs the bf16 emulation {rel_err(out, emulated):.2e} "
              f"(median row {np.median(row_errors(out, emulated)):.1e}), vs the fp32 oracle {err:.2e} "
              f"(median row {np.median(row_errors(out, expect)):.1e})")

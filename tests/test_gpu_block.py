"""GPU parity of the RMSNorm -> Mamba-3 block (x + mixer(GroupedRMSNorm(x)),
python/montlok/rdt/reference/Model/layers/mamba3_layer.py:488-498) and of the
streaming decode chain built from it.

Block: 64 windows x 32 tokens, d_model 64, 4 heads of 32, d_state 16, 8 norm
groups, Kaiming-uniform weights, dt bias per mamba3.py:128-130 -- against the
oracle chain (rms_norm, linear, mamba3_siso_forward, linear + x) at 1e-5, and
against the separate GPU operators bit for bit.

Decode: 2 blocks (d_model 128, d_state 64, 4 heads of 64), RMSNorm, a
Linear(128 -> 1) head; 1024 streams with a started state (ssm, k, v ~
N(0, 0.1), rotary phase ~ U[0, 2 pi)) stepped 3 bars -- against the oracle's
step chain at 1e-5 on the outputs and on every carried state tensor.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import assert_bitwise, assert_close

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


def _init(block, g):
    """nn.Linear's Kaiming-uniform weights; dt_bias with softplus(dt_bias) log-uniform in [1e-3, 1e-1];
    perturbed B/C biases, norms and D so every term carries signal."""
    m = block.mamba
    with torch.no_grad():
        for lin in (m.in_proj, m.out_proj):
            bound = 1 / math.sqrt(lin.in_features)
            lin.weight.copy_((torch.rand(lin.weight.shape, generator=g) * 2 - 1) * bound)
        dt = torch.exp(torch.rand(m.nheads, generator=g) * (math.log(1e-1) - math.log(1e-3)) + math.log(1e-3))
        m.dt_bias.copy_(dt + torch.log(-torch.expm1(-dt)))
        m.B_bias.add_(0.3 * torch.randn(m.B_bias.shape, generator=g))
        m.C_bias.add_(0.3 * torch.randn(m.C_bias.shape, generator=g))
        m.D.add_(0.5 * torch.randn(m.D.shape, generator=g))
        block.norm.weight.normal_(1.0, 0.1, generator=g)


def _oracle_block(oracle, block, x):
    m, nrm = block.mamba, block.norm
    h = oracle.rms_norm(x, _np(nrm.weight), nrm.eps, nrm.num_groups)
    proj = oracle.linear(h, _np(m.in_proj.weight))
    y = oracle.mamba3_siso_forward(proj, m.d_state, m.num_bc_heads, m.nheads, m.headdim, m.num_rope_angles,
                                   _np(m.B_bias), _np(m.C_bias), _np(m.B_norm.weight), _np(m.C_norm.weight),
                                   m.B_norm.eps, m.C_norm.eps, _np(m.dt_bias), _np(m.D), m.A_floor)
    return x + oracle.linear(y, _np(m.out_proj.weight))


@pytest.mark.parametrize("dm,H,groups,B,L", [(64, 4, 8, 64, 32),   # the block workload
                                              (64, 4, 8, 3, 45),    # two chunks, the second partial
                                              (64, 4, 8, 1, 1),
                                              (64, 4, 8, 6, 27),    # one chunk, token tile 1 partial
                                              (64, 4, 8, 4, 12),    # one chunk, token tile 1 past the end
                                              (64, 4, 8, 5, 96),    # three full chunks
                                              (32, 2, 4, 7, 33)])   # d_model 32 in 4 groups of 8, 2 heads
def test_block_vs_oracle_and_separate_ops(dev, oracle, dm, H, groups, B, L):
    """The block (the fused norm + in_proj + scan kernel, then out_proj + x) against the oracle chain at 1e-5
    and against the separate operators bit for bit (they take their one-wave-per-tile linears here)."""
    from montlok import _C
    from montlok.rdt import Mamba3BlockHIP

    g = torch.Generator().manual_seed(B * 100 + L + dm)
    block = Mamba3BlockHIP(dm, d_state=16, expand=2, headdim=32, num_groups=groups).eval()
    assert block.mamba.nheads == H
    _init(block, g)
    x = torch.randn(B, L, dm, generator=g)
    expect = _oracle_block(oracle, block, x.numpy())
    block = block.to(dev)
    xd = x.to(dev)
    with torch.no_grad():
        out = block(xd)
        assert _C.mamba3_block_launches() == ["rms_norm_mamba3_forward", "linear_residual"], "the geometry has the one-launch kernel"
        m = block.mamba
        separate = xd + _C.mamba3_siso_layer(_C.rms_norm(xd, block.norm.weight, 1e-5, groups), m.in_proj.weight,
                                             m.out_proj.weight, *m._mixer_args(), *m._geometry())
    assert out.shape == (B, L, dm)
    assert_close(out, expect, name=f"block {B}x{L} vs oracle")
    assert_bitwise(out, separate.cpu().numpy(), f"block {B}x{L} vs separate operators")


@pytest.mark.parametrize("dm,expand,groups,rope_fraction,B,L", [
    (32, 2, 4, 0.5, 5, 32),     # d_model 32, one chunk: helper waves, weights masked past d_model
    (32, 2, 4, 0.5, 3, 20),     # the same, token tile 1 partial
    (64, 2, 8, 0.0, 4, 32),     # no rotary angles (R = 0), one chunk
    (64, 2, 8, 0.0, 3, 40),     # R = 0, two chunks
    (16, 2, 2, 0.5, 6, 30),     # one head (d_model 16)
    (32, 5, 4, 0.125, 4, 32),   # five heads, one angle: 3H + R = 16, the tile full
    (32, 5, 4, 0.0, 2, 50)])    # five heads, R = 0, two chunks
def test_block_kernel_forms(dev, oracle, dm, expand, groups, rope_fraction, B, L):
    """The mixer kernel's other forms and geometries (d_model below 64 with one-chunk windows, no rotary
    angles, one and five heads): the one-launch block against the oracle chain at 1e-5 and the separate
    operators bit for bit."""
    from montlok import _C
    from montlok.rdt import Mamba3BlockHIP

    g = torch.Generator().manual_seed(B * 1000 + L * 10 + dm + expand)
    block = Mamba3BlockHIP(dm, d_state=16, expand=expand, headdim=32, num_groups=groups,
                           rope_fraction=rope_fraction).eval()
    m = block.mamba
    print(f"block form dm={dm} H={m.nheads} R={m.num_rope_angles} B={B} L={L}", flush=True)
    _init(block, g)
    x = torch.randn(B, L, dm, generator=g)
    expect = _oracle_block(oracle, block, x.numpy())
    block = block.to(dev)
    xd = x.to(dev)
    with torch.no_grad():
        out = block(xd)
        assert _C.mamba3_block_launches() == ["rms_norm_mamba3_forward", "linear_residual"], "the geometry has the one-launch kernel"
        separate = xd + _C.mamba3_siso_layer(_C.rms_norm(xd, block.norm.weight, 1e-5, groups), m.in_proj.weight,
                                             m.out_proj.weight, *m._mixer_args(), *m._geometry())
    assert_close(out, expect, name=f"block form {dm}/{m.nheads}/{m.num_rope_angles} {B}x{L} vs oracle")
    assert_bitwise(out, separate.cpu().numpy(), f"block form {dm}/{m.nheads}/{m.num_rope_angles} {B}x{L} vs separate operators")


def test_block_many_windows_vs_oracle(dev, oracle):
    """300 windows x 70 tokens: 1200 (window, head) blocks of the fused mixer kernel (the separate in_proj
    takes its tiled form here, so only the oracle gate applies)."""
    from montlok import _C
    from montlok.rdt import Mamba3BlockHIP

    g = torch.Generator().manual_seed(77)
    block = Mamba3BlockHIP(64, d_state=16, expand=2, headdim=32, num_groups=8).eval()
    _init(block, g)
    x = torch.randn(300, 70, 64, generator=g)
    expect = _oracle_block(oracle, block, x.numpy())
    block = block.to(dev)
    with torch.no_grad():
        out = block(x.to(dev))
    assert _C.mamba3_block_launches() == ["rms_norm_mamba3_forward", "linear_residual"]
    assert_close(out, expect, name="block 300x70 vs oracle")


def test_block_strided_input_and_unfused_scan(dev, monkeypatch):
    """A token-strided input (a column slice of wider rows) and MLK_MAMBA3_SCAN=unfused, which sends the
    block to the three separate launches with the unfused scan: the same result bit for bit."""
    from montlok import _C
    from montlok.rdt import Mamba3BlockHIP

    g = torch.Generator().manual_seed(78)
    block = Mamba3BlockHIP(64, d_state=16, expand=2, headdim=32, num_groups=8).eval()
    _init(block, g)
    block = block.to(dev)
    wide = torch.randn(7, 40, 96, generator=g).to(dev)
    x = wide[..., 16:80]  # tokens 96 floats apart, windows 40 x 96 apart, dense rows
    assert not x.is_contiguous()
    with torch.no_grad():
        one = block(x)
        assert _C.mamba3_block_launches() == ["rms_norm_mamba3_forward", "linear_residual"]
        monkeypatch.setenv("MLK_MAMBA3_SCAN", "unfused")
        three = block(x.contiguous())
        assert _C.mamba3_block_launches() == ["rms_norm_linear", "mamba3_siso_forward", "linear_residual"]
    assert_bitwise(one, three.cpu().numpy(), "fused mixer vs three launches (unfused scan)")


def _started_states(stack, S, g):
    states = stack.new_state(S)
    for st in states:
        st["ssm"].copy_(torch.randn(st["ssm"].shape, generator=g) * 0.1)
        st["k"].copy_(torch.randn(st["k"].shape, generator=g) * 0.1)
        st["v"].copy_(torch.randn(st["v"].shape, generator=g) * 0.1)
        st["angle"].copy_(torch.rand(st["angle"].shape, generator=g, dtype=torch.float64) * 2 * math.pi)
        st["started"] = True
    return states


def test_decode_chain_vs_oracle(dev, oracle):
    from montlok.rdt import DecodeStackHIP

    g = torch.Generator().manual_seed(21)
    S, T, d = 1024, 3, 128
    stack = DecodeStackHIP(d_model=d, n_layers=2, d_state=64, expand=2, headdim=64, num_groups=8).eval()
    for block in stack.layers:
        _init(block, g)
    with torch.no_grad():
        stack.final_norm.weight.normal_(1.0, 0.1, generator=g)
        stack.head.bias.normal_(0.0, 0.1, generator=g)
    xs = torch.randn(T, S, d, generator=g)
    stack = stack.to(dev)
    states = _started_states(stack, S, g)
    ost = [dict(ssm=_np(s["ssm"]).copy(), k_prev=_np(s["k"]).copy(), v_prev=_np(s["v"]).copy(),
                angle=s["angle"].cpu().numpy().copy(), started=1) for s in states]
    for t in range(T):
        with torch.no_grad():
            out = stack.step(xs[t].to(dev), states)
        h = xs[t].numpy()
        for block, st in zip(stack.layers, ost):
            m, nrm = block.mamba, block.norm
            proj = oracle.linear(oracle.rms_norm(h, _np(nrm.weight), nrm.eps, nrm.num_groups), _np(m.in_proj.weight))
            y = oracle.mamba3_step(proj, st, m.d_state, m.num_bc_heads, m.nheads, m.headdim, m.num_rope_angles,
                                   _np(m.B_bias), _np(m.C_bias), _np(m.B_norm.weight), _np(m.C_norm.weight),
                                   m.B_norm.eps, m.C_norm.eps, _np(m.dt_bias), _np(m.D), m.A_floor)
            h = h + oracle.linear(y, _np(m.out_proj.weight))
        expect = oracle.linear(oracle.rms_norm(h, _np(stack.final_norm.weight), stack.final_norm.eps, 1),
                               _np(stack.head.weight), _np(stack.head.bias))
        assert out.shape == (S, 1)
        assert_close(out, expect, name=f"decode output, bar {t}")
    for i, (st, e) in enumerate(zip(states, ost)):
        assert_close(st["ssm"], e["ssm"], name=f"layer {i} ssm state")
        assert_close(st["k"], e["k_prev"], name=f"layer {i} k state")
        assert_close(st["v"], e["v_prev"], name=f"layer {i} v state")
        np.testing.assert_allclose(st["angle"].cpu().numpy(), e["angle"], rtol=1e-6, atol=1e-6)


def test_decode_full_streams_steps_equal_forward(dev):
    """The decode workload's 65,536 streams (2 blocks, d_model 128, d_state 64, 4 heads of 64): two bars
    stepped from a zero state equal the forward over those two bars to 1e-6 normwise (the step kernel
    against the chunked scan and the tiled linears: a size-independent property at the full size; the
    oracle checks the step chain on 1,024 streams)."""
    from montlok.rdt import DecodeStackHIP

    g = torch.Generator().manual_seed(23)
    stack = DecodeStackHIP(d_model=128, n_layers=2, d_state=64, headdim=64).eval()
    for block in stack.layers:
        _init(block, g)
    stack = stack.to(dev)
    S = 65536
    gd = torch.Generator(device=dev).manual_seed(23)
    x = torch.randn(S, 2, 128, generator=gd, device=dev)
    with torch.no_grad():
        print("decode 65536 streams: forward", flush=True)
        full = stack(x)
        states = stack.new_state(S)
        print("decode 65536 streams: two steps", flush=True)
        steps = torch.stack([stack.step(x[:, t].contiguous(), states) for t in range(2)], dim=1)
    assert torch.isfinite(steps).all()
    assert_close(steps, full, tol=1e-6, name="decode step x 2 vs forward, 65536 streams")


def test_decode_steps_equal_forward(dev):
    """T bars stepped from a zero state give the forward over those T bars, row for row."""
    from montlok.rdt import DecodeStackHIP

    g = torch.Generator().manual_seed(22)
    stack = DecodeStackHIP(d_model=128, n_layers=2, d_state=64, headdim=64).eval()
    for block in stack.layers:
        _init(block, g)
    stack = stack.to(dev)
    x = torch.randn(5, 12, 128, generator=g).to(dev)
    with torch.no_grad():
        full = stack(x)
        states = stack.new_state(5)
        steps = torch.stack([stack.step(x[:, t].contiguous(), states) for t in range(12)], dim=1)
    assert_close(steps, full, tol=1e-6, name="decode step x T vs forward")

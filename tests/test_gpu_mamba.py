"""GPU parity of the Mamba-3 SISO mixer: the recurrence, the fused in_proj
post-processing + recurrence, and the one-token step with carried state.

Against the golden vectors of the compiled reference and the CPU oracle on
the same seeded inputs; gate: normwise relative error <= 1e-5 (fp32). The
forward's one-kernel chunked scan (the default for d_state 16/32/64 and
headdim 16/32/64) equals the unfused prep -> rotate -> chunked-recurrence
kernels bit for bit, and is checked against the time-sequential kernel and
the oracle at 1e-6; so is the recurrent op's chunked scan.
The step is checked against the time-sequential sequence kernel (stepping T
tokens from a zero state equals the forward over T tokens, bit for bit) and
against the oracle's step at the streaming-decode geometry (d_model 128,
d_state 64, 4 heads).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_bitwise, assert_close

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_recurrent_golden(dev, golden):
    from montlok import _C

    g = golden("siso")
    for i in range(4):
        c = {k[len(f"c{i}_"):]: v for k, v in g.items() if k.startswith(f"c{i}_")}
        args = [_t(c[k], dev) for k in ("q", "k", "v", "gate", "adt", "dt", "trap", "skip")]
        out = _C.mamba3_siso_recurrent(*args)
        assert_close(out, c["out"], name=f"siso case {i}")


def _forward_args(c, dev):
    return [_t(c[k], dev) for k in ("b_bias", "c_bias", "b_norm_w", "c_norm_w", "dt_bias", "skip")]


def test_forward_golden(dev, golden):
    from montlok import _C

    g = golden("mamba_forward")
    for i in range(5):
        c = {k[len(f"c{i}_"):]: v for k, v in g.items() if k.startswith(f"c{i}_")}
        N, G, H, D, R = (int(v) for v in c["geom"])
        proj = _t(c["proj"], dev)
        out = _C.mamba3_siso_forward(proj, proj.new_empty(0), *_forward_args(c, dev), N, G, H, D, R, 1e-5, 1e-5, 1e-4)
        assert_close(out, c["out"], name=f"forward case {i} N{N} G{G} H{H} D{D} R{R}")


def _random_layer(rng, B, L, N, G, H, D, R):
    W = 2 * H * D + 2 * G * N + 3 * H + R
    proj = rng.standard_normal((B, L, W)).astype(np.float32)
    params = dict(b_bias=(1 + 0.3 * rng.standard_normal((H, N))).astype(np.float32),
                  c_bias=(1 + 0.3 * rng.standard_normal((H, N))).astype(np.float32),
                  b_norm_w=(rng.random(N) + 0.5).astype(np.float32), c_norm_w=(rng.random(N) + 0.5).astype(np.float32),
                  dt_bias=(rng.standard_normal(H) - 2).astype(np.float32),
                  skip=(rng.standard_normal(H) * 0.5 + 1).astype(np.float32))
    return proj, params


@pytest.mark.parametrize("B,L,N,G,H,D,R", [(64, 32, 16, 1, 4, 32, 4),   # RMSNorm->Mamba-3 block geometry
                                           (2, 256, 64, 1, 8, 64, 16),  # full-stack Mamba geometry, 2 windows
                                           (3, 41, 14, 2, 4, 8, 3),     # grouped B/C, odd N, 8-lane blocks
                                           (2, 19, 6, 1, 3, 12, 1),     # scalar path (headdim 12)
                                           (1, 9, 70, 1, 2, 96, 0)])    # N above 64, headdim above 64
def test_forward_vs_oracle(dev, oracle, B, L, N, G, H, D, R):
    from montlok import _C

    rng = np.random.default_rng(B * L + N)
    proj, p = _random_layer(rng, B, L, N, G, H, D, R)
    plist = [p[k] for k in ("b_bias", "c_bias", "b_norm_w", "c_norm_w", "dt_bias", "skip")]
    expect = oracle.mamba3_siso_forward(proj, N, G, H, D, R, *plist[:4], 1e-5, 1e-5, plist[4], plist[5], 1e-4)
    tp = _t(proj, dev)
    out = _C.mamba3_siso_forward(tp, tp.new_empty(0), *(_t(x, dev) for x in plist), N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    assert_close(out, expect, name="forward")
    # The host libm the reference links (glibc 2.35) rounds fp32 log1pf and
    # tanhf off the correctly rounded value for 1.7% and 13.5% of inputs; the
    # kernel rounds them correctly, so dt, alpha and the rotary phase differ by
    # an ulp now and then and the outputs agree to a few fp32 ulps, not bitwise.
    assert_close(out, expect, tol=1e-6, name="forward (ulp-level agreement)")


def test_forward_strided_projection_and_external_gate(dev, oracle):
    """projected as a slice of a wider buffer (any leading strides), and an explicit gate tensor."""
    from montlok import _C

    rng = np.random.default_rng(7)
    B, L, N, G, H, D, R = 2, 23, 16, 1, 4, 16, 4
    proj, p = _random_layer(rng, B, L, N, G, H, D, R)
    W = proj.shape[-1]
    wide = np.zeros((B, L, W + 24), np.float32)
    wide[:, :, 8:8 + W] = proj
    tw = _t(wide, dev)[:, :, 8:8 + W]
    plist = [_t(p[k], dev) for k in ("b_bias", "c_bias", "b_norm_w", "c_norm_w", "dt_bias", "skip")]
    out = _C.mamba3_siso_forward(tw, tw.new_empty(0), *plist, N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    ref = _C.mamba3_siso_forward(_t(proj, dev), tw.new_empty(0), *plist, N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    assert_bitwise(out, ref.cpu().numpy(), "strided projection")
    z = torch.from_numpy(proj[..., :H * D]).double()
    gate = (z * torch.sigmoid(z)).float().to(dev)
    out_g = _C.mamba3_siso_forward(_t(proj, dev), gate, *plist, N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    assert_close(out_g, ref, tol=2e-6, name="explicit gate vs in-kernel silu")


def test_recurrent_strided_views(dev, oracle):
    """q/k/v/gate as strided views (montlok.cpp:52-55 accepts any leading strides)."""
    from montlok import _C

    rng = np.random.default_rng(9)
    B, L, H, N, D = 2, 17, 3, 16, 32
    big = _t(rng.standard_normal((B, L, H, 2 * N + 2 * D + 5)).astype(np.float32), dev)
    q, k = big[..., :N], big[..., N:2 * N]
    v, gate = big[..., 2 * N:2 * N + D], big[..., 2 * N + D:2 * N + 2 * D]
    dt = torch.nn.functional.softplus(_t(rng.standard_normal((B, L, H)).astype(np.float32), dev) - 2)
    adt = -dt * 0.7
    trap = _t(rng.standard_normal((B, L, H)).astype(np.float32), dev)
    skip = _t(rng.standard_normal(H).astype(np.float32), dev)
    out = _C.mamba3_siso_recurrent(q, k, v, gate, adt, dt, trap, skip)
    al, be, ga = oracle.step_coefficients(adt.cpu().numpy(), dt.cpu().numpy(), trap.cpu().numpy())
    expect = oracle.siso(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), gate.cpu().numpy(), al, be, ga,
                         skip.cpu().numpy())
    assert_close(out, expect, name="strided recurrent")


@pytest.mark.parametrize("N,G,H,D,R", [(16, 1, 4, 16, 4), (64, 1, 4, 64, 16), (6, 1, 3, 12, 1)])
def test_step_equals_sequence(dev, monkeypatch, N, G, H, D, R):
    """T steps equal the time-sequential sequence kernel bit for bit, and the chunked scan to rounding."""
    from montlok import _C

    rng = np.random.default_rng(N + D)
    S, T = 5, 12
    proj, p = _random_layer(rng, S, T, N, G, H, D, R)
    plist = [_t(p[k], dev) for k in ("b_bias", "c_bias", "b_norm_w", "c_norm_w", "dt_bias", "skip")]
    tp = _t(proj, dev)
    chunked = _C.mamba3_siso_forward(tp, tp.new_empty(0), *plist, N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    monkeypatch.setenv("MLK_MAMBA3_SCAN", "sequential")
    seq = _C.mamba3_siso_forward(tp, tp.new_empty(0), *plist, N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    state = _C.new_mamba3_state(S, H, N, D, R, dev)
    for t in range(T):
        y = _C.mamba3_siso_step(tp[:, t].contiguous(), state, *plist, N, G, H, D, R, 1e-5, 1e-5, 1e-4)
        assert_bitwise(y, seq[:, t].cpu().numpy(), f"step {t}")
    assert_close(chunked, seq, tol=1e-6, name="chunked scan vs time-sequential")


@pytest.mark.parametrize("B,L,N,H,D", [(2, 200, 64, 2, 64), (3, 64, 32, 2, 32), (2, 70, 16, 3, 64), (4, 31, 64, 1, 32)])
def test_chunked_scan_vs_sequential(dev, oracle, monkeypatch, B, L, N, H, D):
    """The chunked scan (full, partial and single chunks, both chunk lengths) against the time-sequential
    kernel and the oracle, 1e-6 normwise."""
    from montlok import _C

    rng = np.random.default_rng(L + N)
    R = N // 4
    proj, p = _random_layer(rng, B, L, N, 1, H, D, R)
    plist = [_t(p[k], dev) for k in ("b_bias", "c_bias", "b_norm_w", "c_norm_w", "dt_bias", "skip")]
    tp = _t(proj, dev)
    chunked = _C.mamba3_siso_forward(tp, tp.new_empty(0), *plist, N, 1, H, D, R, 1e-5, 1e-5, 1e-4)
    monkeypatch.setenv("MLK_MAMBA3_SCAN", "sequential")
    seq = _C.mamba3_siso_forward(tp, tp.new_empty(0), *plist, N, 1, H, D, R, 1e-5, 1e-5, 1e-4)
    assert_close(chunked, seq, tol=1e-6, name="chunked vs sequential")
    expect = oracle.mamba3_siso_forward(proj, N, 1, H, D, R, p["b_bias"], p["c_bias"], p["b_norm_w"], p["c_norm_w"],
                                        1e-5, 1e-5, p["dt_bias"], p["skip"], 1e-4)
    assert_close(chunked, expect, tol=1e-6, name="chunked vs oracle")


@pytest.mark.parametrize("B,L,N,G,H,D", [(2, 200, 64, 1, 2, 64), (3, 64, 32, 1, 2, 32), (64, 32, 16, 1, 4, 32),
                                         (2, 70, 16, 1, 3, 64), (4, 31, 64, 2, 2, 32), (8, 33, 32, 2, 4, 64),
                                         (3, 1, 64, 1, 2, 64), (5, 65, 16, 1, 2, 32)])
def test_fused_scan_equals_unfused_chunked(dev, monkeypatch, B, L, N, G, H, D):
    """The one-kernel forward (in_proj post-processing and chunked scan, q/k kept in LDS) equals the
    prep -> rotate -> chunked-recurrence kernels bit for bit: the same arithmetic per token, the same
    matrix-core products in the same order."""
    from montlok import _C

    rng = np.random.default_rng(B + L + N + D)
    R = N // 4 + 1
    proj, p = _random_layer(rng, B, L, N, G, H, D, R)
    plist = [_t(p[k], dev) for k in ("b_bias", "c_bias", "b_norm_w", "c_norm_w", "dt_bias", "skip")]
    tp = _t(proj, dev)
    fused = _C.mamba3_siso_forward(tp, tp.new_empty(0), *plist, N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    monkeypatch.setenv("MLK_MAMBA3_SCAN", "unfused")
    unfused = _C.mamba3_siso_forward(tp, tp.new_empty(0), *plist, N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    assert_bitwise(fused, unfused.cpu().numpy(), "fused vs unfused chunked scan")
    z = tp[..., :H * D].double()
    gate = (z * torch.sigmoid(z)).float()
    monkeypatch.delenv("MLK_MAMBA3_SCAN")
    fused_g = _C.mamba3_siso_forward(tp, gate, *plist, N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    monkeypatch.setenv("MLK_MAMBA3_SCAN", "unfused")
    unfused_g = _C.mamba3_siso_forward(tp, gate, *plist, N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    assert_bitwise(fused_g, unfused_g.cpu().numpy(), "fused vs unfused, explicit gate")


def test_stack_scan_full_size(dev, monkeypatch):
    """The stack's Mamba-3 scan at its full size (1024 windows x 256 tokens, 8 heads of 64, d_state 64, 16
    angles): the fused kernel against the time-sequential kernel (the reference's association) to 1e-6
    normwise and per row; the unfused path (prep -> rotate -> recurrence, which with 8192 window x head
    pairs takes the time-sequential kernel) equals MLK_MAMBA3_SCAN=sequential bit for bit. The oracle
    checks the same geometry on 2 windows (test_forward_vs_oracle); these are its size-independent
    properties."""
    from montlok import _C

    B, L, N, G, H, D, R = 1024, 256, 64, 1, 8, 64, 16
    W = 2 * H * D + 2 * G * N + 3 * H + R
    rng = np.random.default_rng(1024)
    _, p = _random_layer(rng, 1, 1, N, G, H, D, R)
    plist = [_t(p[k], dev) for k in ("b_bias", "c_bias", "b_norm_w", "c_norm_w", "dt_bias", "skip")]
    g = torch.Generator(device=dev).manual_seed(1024)
    tp = torch.randn(B, L, W, generator=g, device=dev)
    print("stack scan 1024 x 256: fused", flush=True)
    fused = _C.mamba3_siso_forward(tp, tp.new_empty(0), *plist, N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    monkeypatch.setenv("MLK_MAMBA3_SCAN", "unfused")
    print("stack scan 1024 x 256: unfused", flush=True)
    unfused = _C.mamba3_siso_forward(tp, tp.new_empty(0), *plist, N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    monkeypatch.setenv("MLK_MAMBA3_SCAN", "sequential")
    print("stack scan 1024 x 256: sequential", flush=True)
    seq = _C.mamba3_siso_forward(tp, tp.new_empty(0), *plist, N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    assert torch.equal(unfused, seq), "unfused vs sequential at 1024 x 256"
    del unfused
    assert torch.isfinite(fused).all()
    err = ((fused - seq).abs().amax() / seq.abs().amax()).item()
    print(f"stack scan 1024 x 256: fused vs sequential {err:.2e} (normwise)", flush=True)
    assert err <= 1e-6, f"fused vs sequential at 1024 x 256: {err:.2e}"
    row = ((fused - seq).abs().amax(-1) / seq.abs().amax()).amax().item()
    assert row <= 1e-6


@pytest.mark.parametrize("B,L,N,G,H,D,R", [(5, 40, 16, 1, 4, 16, 4), (3, 77, 64, 2, 4, 16, 32), (2, 33, 32, 1, 3, 16, 0)])
def test_fused_scan_headdim16_vs_sequential(dev, oracle, monkeypatch, B, L, N, G, H, D, R):
    """headdim 16 (one wave per head, no unfused chunked counterpart), with grouped B/C, every angle
    slot used, and no rotary angles: against the time-sequential kernel and the oracle, 1e-6 normwise."""
    from montlok import _C

    rng = np.random.default_rng(B * L + N)
    proj, p = _random_layer(rng, B, L, N, G, H, D, R)
    plist = [_t(p[k], dev) for k in ("b_bias", "c_bias", "b_norm_w", "c_norm_w", "dt_bias", "skip")]
    tp = _t(proj, dev)
    fused = _C.mamba3_siso_forward(tp, tp.new_empty(0), *plist, N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    monkeypatch.setenv("MLK_MAMBA3_SCAN", "sequential")
    seq = _C.mamba3_siso_forward(tp, tp.new_empty(0), *plist, N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    assert_close(fused, seq, tol=1e-6, name="fused vs sequential")
    expect = oracle.mamba3_siso_forward(proj, N, G, H, D, R, p["b_bias"], p["c_bias"], p["b_norm_w"], p["c_norm_w"],
                                        1e-5, 1e-5, p["dt_bias"], p["skip"], 1e-4)
    assert_close(fused, expect, tol=1e-6, name="fused vs oracle")


@pytest.mark.parametrize("B,L,H,N,D", [(3, 70, 4, 64, 64), (16, 32, 2, 16, 32)])
def test_recurrent_chunked_vs_sequential(dev, oracle, monkeypatch, B, L, H, N, D):
    """mamba3_siso_recurrent on contiguous q/k takes the chunked scan (few window x head pairs);
    against the time-sequential kernel and the oracle, 1e-6 normwise."""
    from montlok import _C

    rng = np.random.default_rng(B * L + H)
    f = lambda *s: _t(rng.standard_normal(s).astype(np.float32), dev)  # noqa: E731
    q, k, v, gate = f(B, L, H, N) * 0.3, f(B, L, H, N) * 0.3, f(B, L, H, D), f(B, L, H, D)
    dt = torch.nn.functional.softplus(f(B, L, H) - 2)
    adt, trap, skip = -dt * 0.7, f(B, L, H), f(H)
    chunked = _C.mamba3_siso_recurrent(q, k, v, gate, adt, dt, trap, skip)
    monkeypatch.setenv("MLK_MAMBA3_SCAN", "sequential")
    seq = _C.mamba3_siso_recurrent(q, k, v, gate, adt, dt, trap, skip)
    assert_close(chunked, seq, tol=1e-6, name="recurrent chunked vs sequential")
    al, be, ga = oracle.step_coefficients(adt.cpu().numpy(), dt.cpu().numpy(), trap.cpu().numpy())
    expect = oracle.siso(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), gate.cpu().numpy(), al, be, ga,
                         skip.cpu().numpy())
    assert_close(chunked, expect, tol=1e-6, name="recurrent chunked vs oracle")


def test_step_decode_geometry_vs_oracle(dev, oracle):
    """Streaming decode geometry: d_model 128 -> d_inner 256, d_state 64, 4 heads, 16 rotary angles."""
    from montlok import _C

    rng = np.random.default_rng(11)
    S, N, G, H, D, R = 2048, 64, 1, 4, 64, 16
    proj, p = _random_layer(rng, S, 1, N, G, H, D, R)
    proj = proj[:, 0]
    plist_np = [p[k] for k in ("b_bias", "c_bias", "b_norm_w", "c_norm_w", "dt_bias", "skip")]
    state_np = dict(ssm=(rng.standard_normal((S, H, N, D)) * 0.1).astype(np.float32),
                    k_prev=(rng.standard_normal((S, H, N)) * 0.1).astype(np.float32),
                    v_prev=(rng.standard_normal((S, H, D)) * 0.1).astype(np.float32),
                    angle=rng.uniform(0, 6, (S, H, R)).astype(np.float64), started=1)
    state = {"ssm": _t(state_np["ssm"], dev), "k": _t(state_np["k_prev"], dev), "v": _t(state_np["v_prev"], dev),
             "angle": _t(state_np["angle"], dev), "started": True}
    y = _C.mamba3_siso_step(_t(proj, dev), state, *(_t(x, dev) for x in plist_np), N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    expect = oracle.mamba3_step(proj, state_np, N, G, H, D, R, *plist_np[:4], 1e-5, 1e-5, plist_np[4], plist_np[5],
                                1e-4)
    assert_close(y, expect, name="step output")
    assert_close(state["ssm"], state_np["ssm"], name="ssm state")
    # k carries the rotary phase, whose tanhf terms glibc rounds off the
    # correctly rounded value now and then: ulp-level, not bitwise.
    assert_close(state["k"], state_np["k_prev"], tol=1e-6, name="k state")
    assert_bitwise(state["v"], state_np["v_prev"], "v state")
    np.testing.assert_allclose(state["angle"].cpu().numpy(), state_np["angle"], rtol=1e-6, atol=1e-6)


def test_mamba_errors(dev):
    from montlok import _C

    proj = torch.zeros(1, 4, 50, device=dev)
    ones = torch.ones(16, device=dev)
    with pytest.raises(RuntimeError, match="does not match the Mamba-3 layout width"):
        _C.mamba3_siso_forward(proj, proj.new_empty(0), torch.ones(32, device=dev), torch.ones(32, device=dev), ones,
                               ones, torch.ones(2, device=dev), torch.ones(2, device=dev), 16, 1, 2, 8, 4, 1e-5, 1e-5,
                               1e-4)
    with pytest.raises(RuntimeError, match="nheads must be divisible by ngroups"):
        _C.mamba3_siso_forward(proj, proj.new_empty(0), ones, ones, ones, ones, ones, ones, 16, 3, 2, 8, 4, 1e-5, 1e-5,
                               1e-4)
    with pytest.raises(RuntimeError, match="num_rope_angles must fit"):
        _C.mamba3_siso_forward(proj, proj.new_empty(0), ones, ones, ones, ones, ones, ones, 16, 1, 2, 8, 9, 1e-5, 1e-5,
                               1e-4)

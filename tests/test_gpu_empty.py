"""Empty batches: every operator accepts zero windows (or rows) and returns an empty result of the right
shape without launching a kernel on an empty grid."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_row_operators_empty(dev):
    from montlok import _C

    x = torch.empty(0, 7, 64, device=dev)
    w = torch.ones(64, device=dev)
    assert _C.rms_norm(x, w, 1e-5, 8).shape == (0, 7, 64)
    res, nrm = _C.add_rms_norm(x, x, w, 1e-5, 1)
    assert res.shape == (0, 7, 64) and nrm.shape == (0, 7, 64)
    assert _C.layer_norm(x, w, None, 1e-5).shape == (0, 7, 64)
    assert _C.swiglu(torch.empty(0, 7, 128, device=dev)).shape == (0, 7, 64)


@pytest.mark.parametrize("wdt", [torch.float32, torch.bfloat16])
def test_linear_family_empty(dev, wdt):
    from montlok import _C

    x = torch.empty(0, 5, 64, device=dev)
    weight = torch.randn(48, 64, device=dev).to(wdt)
    assert _C.linear(x, weight).shape == (0, 5, 48)
    assert _C.linear_residual(x, weight, None, torch.empty(0, 5, 48, device=dev)).shape == (0, 5, 48)
    assert _C.rms_norm_linear(x, torch.ones(64, device=dev), 1e-5, 8, weight).shape == (0, 5, 48)


def test_mhc_empty(dev):
    from montlok import _C

    n, d = 4, 64
    g = torch.Generator().manual_seed(0)
    streams = torch.empty(0, 3, n, d, device=dev)
    nw = torch.ones(d, device=dev)
    pw = (torch.randn(2 * n + n * n, d, generator=g, dtype=torch.float64) / 8).to(dev)
    pb, qb, rb = torch.zeros(n, device=dev), torch.zeros(n, device=dev), torch.zeros(n, n, device=dev)
    a = [torch.tensor(0.5, device=dev) for _ in range(3)]
    agg, pre, post, res = _C.mhc_prepare(streams, nw, 1e-5, pw, pb, qb, rb, *a, 20)
    assert agg.shape == (0, 3, d) and pre.shape == (0, 3, n) and post.shape == (0, 3, n) and res.shape == (0, 3, n, n)
    new = _C.mhc_combine(streams, res, post, agg)
    assert new.shape == (0, 3, n, d)


def test_mamba3_empty(dev):
    from montlok import _C

    N, G, H, D, R = 16, 1, 2, 16, 4
    W = 2 * H * D + 2 * G * N + 3 * H + R
    proj = torch.empty(0, 9, W, device=dev)
    ones = lambda *s: torch.ones(*s, device=dev)  # noqa: E731
    out = _C.mamba3_siso_forward(proj, proj.new_empty(0), ones(H, N), ones(H, N), ones(N), ones(N), ones(H), ones(H),
                                 N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    assert out.shape == (0, 9, H * D)


def test_mhc_combine_prepare_and_collapse_empty(dev):
    from montlok import _C

    n, d = 4, 64
    g = torch.Generator().manual_seed(1)
    streams = torch.empty(0, 3, n, d, device=dev)
    res, post, out = torch.empty(0, 3, n, n, device=dev), torch.empty(0, 3, n, device=dev), torch.empty(0, 3, d, device=dev)
    nw = torch.ones(d, device=dev)
    pw = (torch.randn(2 * n + n * n, d, generator=g, dtype=torch.float64) / 8).to(dev)
    pb, qb, rb = torch.zeros(n, device=dev), torch.zeros(n, device=dev), torch.zeros(n, n, device=dev)
    a = [torch.tensor(0.5, device=dev) for _ in range(3)]
    new, agg, pre, post2, res2 = _C.mhc_combine_prepare(streams, res, post, out, nw, 1e-5, pw, pb, qb, rb, *a, 20)
    assert new.shape == (0, 3, n, d) and agg.shape == (0, 3, d) and res2.shape == (0, 3, n, n)
    assert _C.mhc_combine_collapse(streams, res, post, out).shape[0] == 0


def test_mamba3_step_empty(dev):
    from montlok import _C

    N, G, H, D, R = 16, 1, 2, 16, 4
    W = 2 * H * D + 2 * G * N + 3 * H + R
    ones = lambda *s: torch.ones(*s, device=dev)  # noqa: E731
    state = _C.new_mamba3_state(0, H, N, D, R, dev)
    out = _C.mamba3_siso_step(torch.empty(0, W, device=dev), state, ones(H, N), ones(H, N), ones(N), ones(N), ones(H),
                              ones(H), N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    assert out.shape[0] == 0


@pytest.mark.parametrize("hd,nope,bf16", [(32, 16, True), (32, 16, False), (64, 32, True)])
def test_mla_forward_empty(dev, hd, nope, bf16):
    from montlok import _C
    from test_gpu_mla import rope_tables_t

    H, kvr, L = 4, 64, 8
    d, rope = H * hd, hd - nope
    dt = torch.bfloat16 if bf16 else torch.float32
    x = torch.empty(0, L, d, device=dev)
    in_w = torch.randn(d + kvr + rope, d, device=dev).to(dt)
    up_w = torch.randn(H * (nope + hd), kvr, device=dev).to(dt)
    o_w = torch.randn(d, d, device=dev).to(dt)
    cos, sin = (t.to(dev) for t in rope_tables_t(L, rope))
    out = _C.mla_forward(x, in_w, x.new_empty(0), torch.ones(kvr, device=dev), None, 1e-5, up_w, o_w, cos, sin, H, hd,
                         nope, kvr, L, True, hd ** -0.5)
    assert out.shape == (0, L, d)

"""GPU parity of the mHC residual mix (prepare, combine, collapse, combine_prepare).

HIP results through the C ABI against the golden vectors of the compiled
reference and against the CPU oracle: normwise relative error <= 1e-5 (fp32
outputs), bitwise mismatches reported. At the full mHC benchmark size
(n = 4, d = 128, 8192 tokens, 20 Sinkhorn iterations) the whole output is
compared with the oracle and the Sinkhorn invariants are checked.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_bitwise, assert_close, bit_mismatches

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _params(c, alphas, dev, iters):
    return (_t(c["norm_w"], dev), 1e-5, _t(c["proj_w"], dev), _t(c["pre_bias"], dev), _t(c["post_bias"], dev),
            _t(c["res_bias"], dev), *(torch.tensor(float(a), device=dev) for a in alphas), iters)


def test_mhc_golden(dev, golden):
    from montlok import _C

    g = golden("mhc")
    alphas = [float(v) for v in g["alphas"]]
    for i in range(6):
        c = {k[len(f"c{i}_"):]: v for k, v in g.items() if k.startswith(f"c{i}_")}
        n, d, iters = (int(v) for v in c["meta"])
        p = _params(c, alphas, dev, iters)
        s = _t(c["streams"], dev)
        agg, pre, post, res = _C.mhc_prepare(s, *p)
        for name, a in (("agg", agg), ("pre", pre), ("post", post), ("res", res)):
            assert_close(a, c[name], name=f"case{i} n{n} d{d} {name}")
        agg_n = _C.mhc_prepare(s, *p, 0, _t(c["agg_norm_w"], dev), 1e-6)[0]
        assert_close(agg_n, c["agg_normed"], name=f"case{i} agg_norm")
        back = _C.mhc_prepare(_t(c["streams"][:, :, 0, :], dev), *p, n)
        for name, a in zip(("agg", "pre", "post", "res"), back):
            assert_close(a, c[f"bcast_{name}"], name=f"case{i} broadcast {name}")
        out = _t(c["out"], dev)
        res_in, post_in = _t(c["res"], dev), _t(c["post"], dev)
        new = _C.mhc_combine(s, res_in, post_in, out)
        assert_bitwise(new, c["new"], f"case{i} combine")
        assert_bitwise(_C.mhc_combine_collapse(s, res_in, post_in, out), c["collapsed"], f"case{i} collapse")
        nxt = _C.mhc_combine_prepare(s, res_in, post_in, out, *p)
        assert_bitwise(nxt[0], c["next_new"], f"case{i} combine_prepare streams")
        for name, a in zip(("agg", "pre", "post", "res"), nxt[1:]):
            assert_close(a, c[f"next_{name}"], name=f"case{i} combine_prepare {name}")


def _random_mhc(rng, B, L, n, d):
    s = (rng.standard_normal((B, L, n, d)) * 1.5).astype(np.float32)
    nw = (rng.random(d) + 0.5).astype(np.float32)
    pw = (rng.standard_normal((2 * n + n * n, d)) * 4 / np.sqrt(d)).astype(np.float32).astype(np.float64)
    pb = (rng.standard_normal(n) * 0.5).astype(np.float32)
    qb = (rng.standard_normal(n) * 0.5).astype(np.float32)
    rb = (np.eye(n) * 3 + rng.standard_normal((n, n))).astype(np.float32)
    return s, nw, pw, pb, qb, rb


@pytest.mark.parametrize("B,L,d", [(64, 128, 128), (2, 37, 256), (1, 23, 64), (3, 5, 512)])
def test_mhc_prepare_vs_oracle(dev, oracle, B, L, d):
    from montlok import _C

    n = 4
    rng = np.random.default_rng(d + L)
    s, nw, pw, pb, qb, rb = _random_mhc(rng, B, L, n, d)
    alphas = (0.7, 0.6, 0.8)
    got = _C.mhc_prepare(_t(s, dev), _t(nw, dev), 1e-5, _t(pw, dev), _t(pb, dev), _t(qb, dev), _t(rb, dev),
                         *(torch.tensor(a, device=dev) for a in alphas), 20)
    expect = oracle.mhc_prepare(s, nw, 1e-5, pw, pb, qb, rb, *alphas, 20)
    mism = []
    for name, a, e in zip(("agg", "pre", "post", "res"), got, expect):
        assert_close(a, e, name=name)
        mism.append(bit_mismatches(a, e))
    # Double-precision throughout: the fp32 outputs should agree almost everywhere bit for bit.
    assert sum(mism) <= max(4, B * L * n // 1000), mism
    res = got[3].double()
    assert torch.allclose(res.sum(-2), torch.ones_like(res.sum(-2)), atol=1e-6)


def test_mhc_full_size_vs_oracle(dev, oracle):
    """The mHC benchmark workload: n = 4, d = 128, 8192 tokens, 20 iterations."""
    from montlok import _C

    rng = np.random.default_rng(0)
    n, d, T = 4, 128, 8192
    s, nw, pw, pb, qb, rb = _random_mhc(rng, 64, T // 64, n, d)
    alphas = (0.7, 0.7, 0.7)
    ts = _t(s, dev)
    p = (_t(nw, dev), 1e-5, _t(pw, dev), _t(pb, dev), _t(qb, dev), _t(rb, dev),
         *(torch.tensor(a, device=dev) for a in alphas), 20)
    agg, pre, post, res = _C.mhc_prepare(ts, *p)
    e_agg, e_pre, e_post, e_res = oracle.mhc_prepare(s, nw, 1e-5, pw, pb, qb, rb, *alphas, 20)
    for name, a, e in (("agg", agg, e_agg), ("pre", pre, e_pre), ("post", post, e_post), ("res", res, e_res)):
        assert_close(a, e, name=name)
    out = torch.tanh(agg)
    new = _C.mhc_combine(ts, res, post, out)
    assert_bitwise(new, oracle.mhc_combine(s, res.cpu().numpy(), post.cpu().numpy(), out.cpu().numpy()), "combine")
    # Columns sum to 1 after the final column step; after 20 rounds the rows
    # are only approximately normalised, exactly as far as the oracle's are.
    r = res.double()
    assert (r.sum(-2) - 1).abs().max().item() < 1e-6
    e_rows = torch.from_numpy(e_res.astype(np.float64)).sum(-1)
    assert (r.sum(-1).cpu() - e_rows).abs().max().item() < 1e-6


@pytest.mark.parametrize("n,d", [(4, 128), (3, 64), (8, 32), (9, 20), (4, 66)])
def test_mhc_combine_vs_oracle(dev, oracle, n, d):
    from montlok import _C

    rng = np.random.default_rng(n * d)
    B, L = 3, 17
    s = rng.standard_normal((B, L, n, d)).astype(np.float32)
    res = rng.random((B, L, n, n)).astype(np.float32)
    post = (rng.random((B, L, n)) * 2).astype(np.float32)
    out = rng.standard_normal((B, L, d)).astype(np.float32)
    args = [_t(a, dev) for a in (s, res, post, out)]
    new = _C.mhc_combine(*args)
    assert_bitwise(new, oracle.mhc_combine(s, res, post, out), "combine")
    col = _C.mhc_combine_collapse(*args)
    assert_bitwise(col, oracle.mhc_combine(s, res, post, out, collapse=True, materialize=False), "collapse")
    # Broadcast backbone streams ([B, L, d], stride 0) equal the materialised expand.
    back = s[:, :, 0, :]
    expanded = np.ascontiguousarray(np.broadcast_to(back[:, :, None, :], s.shape))
    got = _C.mhc_combine(_t(back, dev), *args[1:])
    assert_bitwise(got, oracle.mhc_combine(expanded, res, post, out), "broadcast combine")


@pytest.mark.parametrize("d,B,L,agg_norm", [(256, 4, 250, True), (256, 3, 17, False), (128, 5, 200, True),
                                             (128, 2, 9, False), (64, 2, 40, True)])
def test_broadcast_prepare_equals_materialised(dev, d, B, L, agg_norm):
    """The prepare of a broadcast backbone ([B, L, d], stream stride 0: the form specialised to one stream
    load per lane at d 128 and 256) equals the prepare of the materialised expand bit for bit, with and
    without the output RMSNorm of agg."""
    from montlok import _C

    n = 4
    rng = np.random.default_rng(d + B + L)
    s, nw, pw, pb, qb, rb = _random_mhc(rng, B, L, n, d)
    p = (_t(nw, dev), 1e-5, _t(pw, dev), _t(pb, dev), _t(qb, dev), _t(rb, dev),
         *(torch.tensor(v, device=dev) for v in (0.7, 0.6, 0.8)), 20)
    extra = (0, _t((rng.random(d) + 0.5).astype(np.float32), dev), 1e-6) if agg_norm else ()
    backbone = _t(s[:, :, 0, :], dev)
    got = _C.mhc_prepare(backbone, *p, n, *extra[1:]) if agg_norm else _C.mhc_prepare(backbone, *p, n)
    dense_in = backbone.unsqueeze(-2).expand(-1, -1, n, -1).contiguous()
    dense = _C.mhc_prepare(dense_in, *p, *extra) if agg_norm else _C.mhc_prepare(dense_in, *p)
    for name, a, b in zip(("agg", "pre", "post", "res"), got, dense):
        assert_bitwise(a, b.cpu().numpy(), f"broadcast {name} d{d} {B}x{L}")


def test_mhc_combine_prepare_equals_separate_passes(dev):
    """The fused write+read equals combine then prepare bit for bit (montlok_selftest.cpp:606-677)."""
    from montlok import _C

    rng = np.random.default_rng(12)
    n, d = 4, 64
    s, nw, pw, pb, qb, rb = _random_mhc(rng, 2, 19, n, d)
    p = (_t(nw, dev), 1e-5, _t(pw, dev), _t(pb, dev), _t(qb, dev), _t(rb, dev),
         *(torch.tensor(0.6, device=dev) for _ in range(3)), 7)
    backbone = _t(s[:, :, 0, :], dev)
    agg, pre, post, res = _C.mhc_prepare(backbone, *p, n)
    dense = _C.mhc_prepare(backbone.unsqueeze(-2).expand(-1, -1, n, -1).contiguous(), *p)
    for a, b in zip((agg, pre, post, res), dense):
        assert_bitwise(a, b.cpu().numpy(), "broadcast prepare == materialised prepare")
    out = torch.tanh(agg)
    fused = _C.mhc_combine_prepare(backbone, res, post, out, *p)
    sep_streams = _C.mhc_combine(backbone, res, post, out)
    sep = _C.mhc_prepare(sep_streams, *p)
    assert_bitwise(fused[0], sep_streams.cpu().numpy(), "streams")
    for a, b in zip(fused[1:], sep):
        assert_bitwise(a, b.cpu().numpy(), "coefficients")
    collapsed = _C.mhc_combine_collapse(fused[0], fused[4], fused[3], torch.tanh(fused[1]))
    materialized = _C.mhc_combine(fused[0], fused[4], fused[3], torch.tanh(fused[1]))
    assert_close(collapsed, materialized.double().mean(-2).float(), tol=3e-7)


def test_mhc_errors(dev):
    from montlok import _C

    s = torch.zeros(1, 4, 4, 8, device=dev)
    ok = dict(norm_w=torch.ones(8, device=dev), eps=1e-5, proj_w=torch.zeros(24, 8, device=dev, dtype=torch.float64),
              pre_bias=torch.zeros(4, device=dev), post_bias=torch.zeros(4, device=dev),
              res_bias=torch.zeros(16, device=dev), pre_alpha=torch.tensor(0.0, device=dev),
              post_alpha=torch.tensor(0.0, device=dev), res_alpha=torch.tensor(0.0, device=dev), sinkhorn_iters=3)
    with pytest.raises(RuntimeError, match="sinkhorn_iters must be non-negative"):
        _C.mhc_prepare(s, **{**ok, "sinkhorn_iters": -1})
    with pytest.raises(RuntimeError, match="proj_w must be a contiguous float64"):
        _C.mhc_prepare(s, **{**ok, "proj_w": torch.zeros(24, 8, device=dev)})
    with pytest.raises(RuntimeError, match="n_streams is required"):
        _C.mhc_prepare(s[:, :, 0].contiguous(), **ok)
    # The stream count comes from res (montlok.cpp:730), checked before res itself.
    with pytest.raises(RuntimeError, match="streams has 4 streams, expected 3"):
        _C.mhc_combine(s, torch.zeros(1, 4, 3, 3, device=dev), torch.zeros(1, 4, 4, device=dev),
                       torch.zeros(1, 4, 8, device=dev))
    with pytest.raises(RuntimeError, match="res must be contiguous"):
        _C.mhc_combine(s, torch.zeros(1, 4, 4, 4, device=dev).transpose(2, 3), torch.zeros(1, 4, 4, device=dev),
                       torch.zeros(1, 4, 8, device=dev))


def test_mhc_combine_prepare_plain_store_branch(dev, oracle):
    """Above 65,536 tokens the fused combine+prepare stores its outputs with plain (not non-temporal)
    stores. At 70,000 tokens x d 256 x n 4 it equals combine then prepare bit for bit, and a 1,024-token
    slice matches the oracle (montlok_selftest.cpp:606-677)."""
    from montlok import _C

    rng = np.random.default_rng(70000)
    n, d, B, L = 4, 256, 70, 1000
    s, nw, pw, pb, qb, rb = _random_mhc(rng, B, L, n, d)
    alphas = (0.7, 0.6, 0.8)
    p = (_t(nw, dev), 1e-5, _t(pw, dev), _t(pb, dev), _t(qb, dev), _t(rb, dev),
         *(torch.tensor(a, device=dev) for a in alphas), 20)
    ts = _t(s, dev)
    agg, pre, post, res = _C.mhc_prepare(ts, *p)
    out = torch.tanh(agg)
    fused = _C.mhc_combine_prepare(ts, res, post, out, *p)
    sep_streams = _C.mhc_combine(ts, res, post, out)
    sep = _C.mhc_prepare(sep_streams, *p)
    assert fused[0].shape == (B, L, n, d)
    assert_bitwise(fused[0], sep_streams.cpu().numpy(), "streams, 70,000 tokens")
    for name, a, b in zip(("agg", "pre", "post", "res"), fused[1:], sep):
        assert_bitwise(a, b.cpu().numpy(), f"{name}, 70,000 tokens")
    # The oracle on a 1,024-token slice: the first 1,024 tokens of windows 37 and 38.
    w0 = 37
    s_sl = s[w0:w0 + 2]
    res_sl, post_sl, out_sl = (t[w0:w0 + 2].cpu().numpy() for t in (res, post, out))
    e_new = oracle.mhc_combine(s_sl, res_sl, post_sl, out_sl)
    e_prep = oracle.mhc_prepare(e_new, nw, 1e-5, pw, pb, qb, rb, *alphas, 20)
    flat = lambda a: a.reshape(2 * L, *a.shape[2:])[:1024]  # noqa: E731
    assert_bitwise(flat(fused[0][w0:w0 + 2].cpu().numpy()), flat(e_new), "streams vs oracle, 1,024 tokens")
    mism = 0
    for name, a, e in zip(("agg", "pre", "post", "res"), fused[1:], e_prep):
        a_sl = flat(a[w0:w0 + 2].cpu().numpy())
        assert_close(a_sl, flat(np.asarray(e)), name=f"{name} vs oracle")
        mism += bit_mismatches(a_sl, flat(np.asarray(e)))
    assert mism <= max(4, 1024 * n // 1000), mism


@pytest.mark.parametrize("n,d,B,L", [(4, 128, 3, 50), (4, 256, 2, 33), (4, 512, 2, 9), (3, 64, 2, 21), (8, 32, 1, 17),
                                     (5, 18, 2, 7)])
def test_combine_prepare_in_place_and_reused_buffers(dev, n, d, B, L):
    """The stage-2 buffer variants (montlok.cpp:807-912): new streams written over the old ones and the next
    residual's coefficients over the current res/post (and agg over out) give the out-of-place values bit for
    bit, through the fused kernel (n = 4, d <= 256) and through combine then prepare (the other shapes)."""
    from montlok import _C

    rng = np.random.default_rng(n * d + L)
    s, nw, pw, pb, qb, rb = _random_mhc(rng, B, L, n, d)
    p = (_t(nw, dev), 1e-5, _t(pw, dev), _t(pb, dev), _t(qb, dev), _t(rb, dev),
         *(torch.tensor(a, device=dev) for a in (0.7, 0.6, 0.8)), 20)
    streams = _t(s, dev)
    agg, pre, post, res = _C.mhc_prepare(streams, *p)
    out = torch.tanh(agg)
    expect = _C.mhc_combine_prepare(streams, res, post, out, *p)
    work = [streams.clone(), agg.clone(), pre.clone(), post.clone(), res.clone(), out.clone()]
    got = _C._mhc_combine_prepare(work[0], work[4], work[3], work[5], *p, reuse_streams=True,
                                  into=(work[5], work[2], work[3], work[4]))
    assert got[0].data_ptr() == work[0].data_ptr() and got[1].data_ptr() == work[5].data_ptr()
    for name, a, b in zip(("streams", "agg", "pre", "post", "res"), got, expect):
        assert_bitwise(a, b.cpu().numpy(), f"in place {name} n{n} d{d}")
    # mhc_combine in place as well
    moved = streams.clone()
    _C._call("mlk_mhc_combine", moved.data_ptr(), B * L, n, d, d, n * d, res.data_ptr(), post.data_ptr(),
             out.data_ptr(), moved.data_ptr(), None, _C._stream())
    assert_bitwise(moved, _C.mhc_combine(streams, res, post, out).cpu().numpy(), f"combine in place n{n} d{d}")


def test_in_place_rejects_strided_streams(dev):
    from montlok import _C

    s = torch.zeros(1, 4, 4, 16, device=dev)
    wide = torch.zeros(1, 4, 4, 24, device=dev)[..., :16]
    res, post, out = torch.zeros(1, 4, 4, 4, device=dev), torch.zeros(1, 4, 4, device=dev), torch.zeros(1, 4, 16,
                                                                                                          device=dev)
    lib = _C.library()
    st = lib.mlk_mhc_combine(wide.data_ptr(), 4, 4, 16, 24, 96, res.data_ptr(), post.data_ptr(), out.data_ptr(),
                             wide.data_ptr(), None, _C._stream())
    assert st == 1 and "in-place mhc_combine needs contiguous" in lib.mlk_last_error().decode()
    st = lib.mlk_mhc_combine(s.data_ptr(), 4, 4, 16, 16, 64, res.data_ptr(), post.data_ptr(), out.data_ptr(),
                             s.data_ptr(), None, _C._stream())
    assert st == 0

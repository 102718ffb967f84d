"""GPU parity of MLA: the rotary key assembly (mla_rope_qk), the attention
contraction, and the whole mla_forward block.

mla_rope_qk is fp64 arithmetic rounded once, the same operations as the
reference kernel, so it is compared bit for bit with the reference's golden
vectors and the oracle. Attention and mla_forward are compared with the
oracle's float64 softmax attention (which itself is pinned against torch in
float64): fp32 precision and fp32 weights within 1e-5, bf16 precision and
bf16 weights within 2e-2 (normwise relative).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import bf16_emu as emu
from helpers import BF16_TOL, assert_bitwise, assert_close, assert_emulated, rel_err, row_errors

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def rope_tables(length: int, rope_dim: int, theta: float = 10000.0):
    """Token-index RoPE tables as the reference builds them with torch on the CPU
    (reference/Model/layers/rope.py:9-16, 138-166): cat(angles, angles)."""
    idx = torch.arange(0, rope_dim, 2, dtype=torch.float32)
    freqs = 1.0 / (theta ** (idx / rope_dim))
    pos = torch.arange(0, length, dtype=torch.float32)
    angles = pos.unsqueeze(-1) * freqs.unsqueeze(0)
    emb = torch.cat([angles, angles], dim=-1)
    return emb.cos().numpy(), emb.sin().numpy()


def test_rope_golden(dev, golden):
    from montlok import _C

    g = golden("rope")
    cases = sorted({k.split("_")[0] for k in g})
    for c in cases:
        case = {k[len(c) + 1:]: v for k, v in g.items() if k.startswith(c + "_")}
        nope = int(case["nope"][0])
        q = _t(case["q"], dev)
        k = _C.mla_rope_qk(q, _t(case["kv"], dev), _t(case["k_rope"], dev), _t(case["cos"], dev),
                           _t(case["sin"], dev), nope)
        assert_bitwise(q, case["q_out"], f"{c} q")
        assert_bitwise(k, case["k_out"], f"{c} k")


@pytest.mark.parametrize("B,L,Lq,H,hd,nope", [(4, 128, 128, 8, 32, 16), (2, 256, 256, 4, 64, 32),
                                              (3, 19, 5, 3, 12, 4), (2, 33, 1, 2, 64, 0)])
def test_rope_vs_oracle_column_slices(dev, oracle, B, L, Lq, H, hd, nope):
    """q and k_rope as column slices of one fused projection output (montlok.cpp:1109-1118)."""
    from montlok import _C

    rng = np.random.default_rng(B * L + hd)
    rope = hd - nope
    kv_rank = 16
    W = H * hd + kv_rank + rope
    proj = rng.standard_normal((B, L, W)).astype(np.float32)
    kv = rng.standard_normal((B, L, H, nope + hd)).astype(np.float32)
    cos, sin = rope_tables(L, rope)
    tproj = _t(proj, dev)
    q_full = tproj[:, L - Lq:, :H * hd]
    q = torch.empty((B, Lq, H * hd), device=dev)
    q.copy_(q_full)
    q = q.view(B, Lq, H, hd) if Lq != L else q_full.unflatten(-1, (H, hd))
    k_rope = tproj[..., H * hd + kv_rank:]
    k = _C.mla_rope_qk(q, _t(kv, dev), k_rope, _t(cos, dev), _t(sin, dev), nope)
    q_exp, k_exp = oracle.mla_rope(proj[:, L - Lq:, :H * hd].reshape(B, Lq, H, hd), kv, proj[..., H * hd + kv_rank:],
                                   cos, sin, nope)
    assert_bitwise(k, k_exp, "k")
    assert_bitwise(q, q_exp, "q rotated in place")


ATTN_CASES = [  # B, Lq, Lk, H, hd, mask
    (3, 128, 128, 8, 32, 1),   # MLA block geometry, causal
    (2, 256, 256, 4, 64, 1),   # full-stack MLA geometry
    (2, 200, 200, 2, 48, 1),   # ragged length, hd padded inside the kernel
    (2, 1, 77, 3, 32, 0),      # one trailing query sees every key
    (2, 5, 77, 3, 16, 2),      # several trailing queries, bottom-right mask
    (1, 130, 130, 1, 128, 0),  # widest head, no mask
    (2, 480, 480, 2, 64, 1),   # the deployed sequence length
]


@pytest.mark.parametrize("B,Lq,Lk,H,hd,mask", ATTN_CASES)
@pytest.mark.parametrize("precision", [torch.float32, torch.bfloat16])
def test_attention_vs_oracle(dev, oracle, B, Lq, Lk, H, hd, mask, precision):
    from montlok import _C

    rng = np.random.default_rng(B + Lq + Lk + hd + mask)
    q = rng.standard_normal((B, Lq, H, hd)).astype(np.float32)
    k = rng.standard_normal((B, Lk, H, hd)).astype(np.float32)
    v = rng.standard_normal((B, Lk, H, hd)).astype(np.float32)
    scale = 1.0 / math.sqrt(hd)
    out = _C.attention(_t(q, dev), _t(k, dev), _t(v, dev), mask, scale, precision)
    expect = oracle.sdpa(q, k, v, mask, scale)
    tol = 1e-5 if precision == torch.float32 else BF16_TOL
    assert_close(out, expect, tol=tol, name=f"attention {precision}")


def test_attention_strided_views(dev, oracle):
    """q as a column slice of a projection, v as the tail of each kv head (mla_forward's views)."""
    from montlok import _C

    rng = np.random.default_rng(17)
    B, L, H, hd, nope = 3, 70, 4, 32, 16
    proj = _t(rng.standard_normal((B, L, H * hd + 40)).astype(np.float32), dev)
    q = proj[..., :H * hd].unflatten(-1, (H, hd))
    kv = _t(rng.standard_normal((B, L, H, nope + hd)).astype(np.float32), dev)
    v = kv[..., nope:]
    k = _t(rng.standard_normal((B, L, H, hd)).astype(np.float32), dev)
    out = _C.attention(q, k, v, _C.MASK_CAUSAL_TOP_LEFT, 0.2)
    expect = oracle.sdpa(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), 1, 0.2)
    assert_close(out, expect, name="strided attention")


def _mla_params(rng, d, H, hd, nope, kv_rank, bf16):
    rope = hd - nope
    std = 0.02 if bf16 else 1 / math.sqrt(d)
    p = dict(q=rng.standard_normal((H * hd, d)) * std, kv_down=rng.standard_normal((kv_rank, d)) * std,
             k_rope=rng.standard_normal((rope, d)) * std,
             kv_up=rng.standard_normal((H * (nope + hd), kv_rank)) * (0.02 if bf16 else 1 / math.sqrt(kv_rank)),
             o=rng.standard_normal((d, H * hd)) * (0.02 if bf16 else 1 / math.sqrt(H * hd)))
    p = {k: v.astype(np.float32) for k, v in p.items()}
    if bf16:
        p = {k: torch.from_numpy(v).bfloat16().float().numpy() for k, v in p.items()}
    p["ln_w"] = (1 + 0.1 * rng.standard_normal(kv_rank)).astype(np.float32)
    p["ln_b"] = (0.1 * rng.standard_normal(kv_rank)).astype(np.float32)
    return p


def _oracle_mla(oracle, x, p, H, hd, nope, kv_rank, n_last, causal, scale, cos, sin):
    B, L, d = x.shape
    in_w = np.concatenate([p["q"], p["kv_down"], p["k_rope"]]) if n_last == L else np.concatenate(
        [p["kv_down"], p["k_rope"]])
    projected = oracle.linear(x, in_w)
    qw = d if n_last == L else 0
    q = projected[..., :qw] if n_last == L else oracle.linear(x[:, L - 1:], p["q"])
    q = q.reshape(B, n_last, H, hd)
    kv_lat = projected[..., qw:qw + kv_rank]
    k_rope = projected[..., qw + kv_rank:]
    kv = oracle.linear(oracle.layer_norm(kv_lat, p["ln_w"], p["ln_b"], 1e-5), p["kv_up"]).reshape(B, L, H, nope + hd)
    q, k = oracle.mla_rope(q, kv, k_rope, cos, sin, nope)
    att = oracle.sdpa(q, k, np.ascontiguousarray(kv[..., nope:]), 1 if (n_last == L and causal) else 0, scale)
    return oracle.linear(att.reshape(B, n_last, d), p["o"])


MLA_GEOMETRIES = {
    # MLA block: d_model 256, 8 heads of 32 (rope 16, nope 16), kv rank 64, 128 tokens; 16 windows.
    "block": (16, 128, 256, 8, 32, 16, 64),
    # Full stack's MLA: d_model 256, 4 heads of 64 (rope 32, nope 32), kv rank 64, 256 tokens; 8 windows.
    "stack": (8, 256, 256, 4, 64, 32, 64),
}


@pytest.mark.parametrize("geometry", sorted(MLA_GEOMETRIES))
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("n_last", ["full", 1])
def test_mla_forward_block_geometry(dev, oracle, bf16, n_last, geometry):
    """mla_forward (the fused attend kernels where built) against the oracle chain at each geometry."""
    from montlok import _C

    rng = np.random.default_rng(1 + bf16)
    B, L, d, H, hd, nope, kv_rank = MLA_GEOMETRIES[geometry]
    n_last = L if n_last == "full" else n_last
    x = rng.standard_normal((B, L, d)).astype(np.float32)
    p = _mla_params(rng, d, H, hd, nope, kv_rank, bf16)
    cos, sin = rope_tables(L, hd - nope)
    scale = 1.0 / math.sqrt(hd)
    wdt = torch.bfloat16 if bf16 else torch.float32

    def w(a):
        return _t(a, dev).to(wdt)

    in_w = np.concatenate([p["q"], p["kv_down"], p["k_rope"]]) if n_last == L else np.concatenate(
        [p["kv_down"], p["k_rope"]])
    q_w = w(p["q"]) if n_last == 1 else torch.empty(0, device=dev)
    out = _C.mla_forward(_t(x, dev), w(in_w), q_w, _t(p["ln_w"], dev), _t(p["ln_b"], dev), 1e-5, w(p["kv_up"]),
                         w(p["o"]), _t(cos, dev), _t(sin, dev), H, hd, nope, kv_rank, n_last, True, scale)
    assert out.shape == (B, n_last, d)
    expect = _oracle_mla(oracle, x, p, H, hd, nope, kv_rank, n_last, True, scale, cos, sin)
    assert_close(out, expect, tol=BF16_TOL if bf16 else 1e-5,
                 name=f"mla_forward {geometry} bf16={bf16} n_last={n_last}")


def test_mla_errors(dev):
    from montlok import _C

    x = torch.zeros(2, 8, 64, device=dev)
    w = torch.zeros(64 + 16 + 8, 64, device=dev)
    with pytest.raises(RuntimeError, match="invalid MLA head geometry"):
        _C.mla_forward(x, w, x.new_empty(0), torch.ones(16, device=dev), None, 1e-5, w, w, w, w, 3, 16, 8, 16, 8,
                       True, 0.25)
    with pytest.raises(RuntimeError, match="native MLA supports the final query or the full sequence"):
        _C.mla_forward(x, w, x.new_empty(0), torch.ones(16, device=dev), None, 1e-5, w, w, w, w, 4, 16, 8, 16, 3,
                       True, 0.25)
    q = torch.zeros(1, 4, 2, 16, device=dev)
    kv = torch.zeros(1, 4, 2, 24, device=dev)
    with pytest.raises(RuntimeError, match="positive even rope_dim"):
        _C.mla_rope_qk(q, kv, torch.zeros(1, 4, 7, device=dev), torch.zeros(4, 7, device=dev),
                       torch.zeros(4, 7, device=dev), 9)
    with pytest.raises(RuntimeError, match="k_rope must be \\[B,L,rope_dim\\]"):
        _C.mla_rope_qk(q, kv, torch.zeros(1, 4, 6, device=dev), torch.zeros(4, 8, device=dev),
                       torch.zeros(4, 8, device=dev), 8)


@pytest.mark.parametrize("B,L,H,hd,nope", [(16, 128, 8, 32, 16),   # MLA block geometry
                                           (8, 256, 4, 64, 32),    # full-stack MLA geometry
                                           (3, 100, 8, 32, 16),    # windows not a multiple of 8, ragged length
                                           (2, 77, 4, 64, 32),
                                           (48, 128, 8, 32, 16), (60, 100, 8, 32, 16)])
def test_fused_attend_equals_separate_kernels(dev, B, L, H, hd, nope):
    """With bf16 weights the full causal mla_forward runs LayerNorm, kv_up, RoPE and attention in one
    kernel; it must give the separate kernels' result bit for bit."""
    from montlok import _C

    g = torch.Generator().manual_seed(B * L + hd)
    d, kvr, rope = H * hd, 64, hd - nope
    bf = torch.bfloat16
    x = torch.randn(B, L, d, generator=g).to(dev)
    in_w = (torch.randn(d + kvr + rope, d, generator=g) * 0.02).to(dev, bf)
    up_w = (torch.randn(H * (nope + hd), kvr, generator=g) * 0.02).to(dev, bf)
    o_w = (torch.randn(d, d, generator=g) * 0.02).to(dev, bf)
    ln_w = (1 + 0.1 * torch.randn(kvr, generator=g)).to(dev)
    ln_b = (0.1 * torch.randn(kvr, generator=g)).to(dev)
    cos, sin = (t.to(dev) for t in rope_tables_t(L, rope))
    args = (x, in_w, x.new_empty(0), ln_w, ln_b, 1e-5, up_w, o_w, cos, sin, H, hd, nope, kvr, L, True, hd ** -0.5)
    fused = _C._mla_forward(*args, allow_fused=True)
    separate = _C._mla_forward(*args, allow_fused=False)
    assert_bitwise(fused, separate.cpu().numpy(), "fused vs separate MLA attention")


def rope_tables_t(length: int, rope_dim: int):
    cos, sin = rope_tables(length, rope_dim)
    return torch.from_numpy(cos), torch.from_numpy(sin)


@pytest.mark.parametrize("B,L,H,hd,nope", [(16, 128, 8, 32, 16), (8, 256, 4, 64, 32), (3, 100, 8, 32, 16),
                                           (2, 77, 4, 64, 32)])
def test_latent_layernorm_once_per_row(dev, B, L, H, hd, nope):
    """The latent LayerNorm'd once per row into bf16 feeds the attention that skips its own LayerNorm: the
    result equals the attention that normalises in every head's block, bit for bit."""
    from montlok import _C

    g = torch.Generator().manual_seed(B + L + hd)
    d, kvr, rope = H * hd, 64, hd - nope
    bf = torch.bfloat16
    x = torch.randn(B, L, d, generator=g).to(dev)
    in_w = (torch.randn(d + kvr + rope, d, generator=g) * 0.02).to(dev, bf)
    up_w = (torch.randn(H * (nope + hd), kvr, generator=g) * 0.02).to(dev, bf)
    ln_w = (1 + 0.1 * torch.randn(kvr, generator=g)).to(dev)
    ln_b = (0.1 * torch.randn(kvr, generator=g)).to(dev)
    cos, sin = (t.to(dev) for t in rope_tables_t(L, rope))
    att = _C._fused_attend_ln(x, in_w, B, L, d, H, hd, nope, kvr, ln_w, ln_b, 1e-5, up_w, cos, sin, hd ** -0.5)
    assert att is not None, "the geometry has the fused kernels"
    projected = _C.linear(x, in_w)
    ref = _C._fused_attend(projected, B, L, d, H, hd, nope, kvr, ln_w, ln_b, 1e-5, up_w, cos, sin, hd ** -0.5)
    assert torch.equal(att, ref)


@pytest.mark.parametrize("B,L,bias,strided", [(16, 128, True, False),   # MLA block geometry
                                              (3, 37, True, False), (2, 1, False, False), (5, 64, False, True),
                                              (1, 127, True, True), (64, 128, True, False), (9, 100, False, False),
                                              (256, 128, True, False)])  # the MLA workload's full 256 windows
def test_window_kernel_equals_separate_path(dev, B, L, bias, strided):
    """With bf16 weights, 8 heads of 32 and L <= 128 the whole mla_forward is one launch, one block per
    window: the result equals the four-launch path (linear, latent LayerNorm into bf16, fused attention,
    linear) bit for bit, for ragged lengths, no kv_norm bias and token-strided x."""
    from montlok import _C

    g = torch.Generator().manual_seed(B * 1000 + L)
    H, hd, nope, kvr = 8, 32, 16, 64
    d, rope = H * hd, hd - nope
    bf = torch.bfloat16
    wide = torch.randn(B, L, d + 64 if strided else d, generator=g).to(dev)
    x = wide[..., 32:32 + d] if strided else wide
    in_w = (torch.randn(d + kvr + rope, d, generator=g) * 0.05).to(dev, bf)
    up_w = (torch.randn(H * (nope + hd), kvr, generator=g) * 0.1).to(dev, bf)
    o_w = (torch.randn(d, d, generator=g) * 0.05).to(dev, bf)
    ln_w = (1 + 0.1 * torch.randn(kvr, generator=g)).to(dev)
    ln_b = (0.1 * torch.randn(kvr, generator=g)).to(dev) if bias else None
    cos, sin = (t.to(dev) for t in rope_tables_t(L, rope))
    args = (x, in_w, x.new_empty(0), ln_w, ln_b, 1e-5, up_w, o_w, cos, sin, H, hd, nope, kvr, L, True, hd ** -0.5)
    one = _C._mla_forward(*args, allow_fused=True)
    assert _C.mla_forward_launches() == ["mla_forward"], "the geometry has the per-window kernel"
    four = _C._mla_forward(*args, allow_fused=True, allow_window=False)
    assert _C.mla_forward_launches() == ["linear", "layer_norm_bf16", "mla_attend_normed", "linear"]
    assert one.shape == (B, L, d)
    assert_bitwise(one, four.cpu().numpy(), f"per-window MLA {B}x{L} vs four launches")


@pytest.mark.parametrize("B,L,bias,strided", [(8, 256, True, False),   # full-stack MLA geometry
                                              (3, 77, True, False), (2, 1, False, False), (5, 64, False, True),
                                              (1, 255, True, True), (16, 200, True, False), (9, 130, False, False),
                                              (4, 65, True, False),
                                              (1024, 256, True, False)])  # the stack's full 1024 windows
def test_span_kernel_equals_separate_path(dev, B, L, bias, strided):
    """With bf16 weights, 4 heads of 64 (rope 32) and L <= 256 the whole mla_forward is one launch, one
    block per (window, 64 query rows) walking the key rows up to them: the result equals the four-launch
    path bit for bit, for ragged lengths (one to four spans, partial last spans), windows not a multiple
    of 8, no kv_norm bias and token-strided x."""
    from montlok import _C

    g = torch.Generator().manual_seed(B * 1000 + L + 5)
    H, hd, nope, kvr = 4, 64, 32, 64
    d, rope = H * hd, hd - nope
    bf = torch.bfloat16
    wide = torch.randn(B, L, d + 64 if strided else d, generator=g).to(dev)
    x = wide[..., 32:32 + d] if strided else wide
    in_w = (torch.randn(d + kvr + rope, d, generator=g) * 0.05).to(dev, bf)
    up_w = (torch.randn(H * (nope + hd), kvr, generator=g) * 0.1).to(dev, bf)
    o_w = (torch.randn(d, d, generator=g) * 0.05).to(dev, bf)
    ln_w = (1 + 0.1 * torch.randn(kvr, generator=g)).to(dev)
    ln_b = (0.1 * torch.randn(kvr, generator=g)).to(dev) if bias else None
    cos, sin = (t.to(dev) for t in rope_tables_t(L, rope))
    args = (x, in_w, x.new_empty(0), ln_w, ln_b, 1e-5, up_w, o_w, cos, sin, H, hd, nope, kvr, L, True, hd ** -0.5)
    print(f"span kernel case B={B} L={L} bias={bias} strided={strided}", flush=True)
    one = _C._mla_forward(*args, allow_fused=True)
    assert _C.mla_forward_launches() == ["mla_forward"], "the geometry has the per-span kernel"
    four = _C._mla_forward(*args, allow_fused=True, allow_window=False)
    assert _C.mla_forward_launches() == ["linear", "layer_norm_bf16", "mla_attend_normed", "linear"]
    assert one.shape == (B, L, d)
    assert_bitwise(one, four.cpu().numpy(), f"per-span MLA {B}x{L} vs four launches")


@pytest.mark.parametrize("B,L,H,hd,nope", [(6, 100, 8, 32, 16), (5, 200, 4, 64, 32)])
def test_packed_weights_equal_row_major(dev, B, L, H, hd, nope):
    """_C.mla_forward runs the one-launch kernel on its weights re-laid in the kernel's fragment order
    (mlk_mla_pack_weights, cached per weight triple): the result equals mlk_mla_forward on the row-major
    weights bit for bit, and the packed copy follows an in-place update of a weight."""
    from montlok import _C

    g = torch.Generator().manual_seed(7 + H)
    kvr = 64
    d, rope = H * hd, hd - nope
    bf = torch.bfloat16
    x = torch.randn(B, L, d, generator=g).to(dev)
    in_w = (torch.randn(d + kvr + rope, d, generator=g) * 0.05).to(dev, bf)
    up_w = (torch.randn(H * (nope + hd), kvr, generator=g) * 0.1).to(dev, bf)
    o_w = (torch.randn(d, d, generator=g) * 0.05).to(dev, bf)
    ln_w = (1 + 0.1 * torch.randn(kvr, generator=g)).to(dev)
    ln_b = (0.1 * torch.randn(kvr, generator=g)).to(dev)
    cos, sin = (t.to(dev) for t in rope_tables_t(L, rope))
    scale = hd ** -0.5
    lib = _C.library()

    def row_major():
        out = torch.empty(B, L, d, device=dev)
        status = lib.mlk_mla_forward(x.data_ptr(), B, L, d, x.stride(0), x.stride(1), in_w.data_ptr(),
                                     ln_w.data_ptr(), ln_b.data_ptr(), 1e-5, up_w.data_ptr(), o_w.data_ptr(),
                                     cos.data_ptr(), sin.data_ptr(), H, hd, nope, kvr, 1, scale, out.data_ptr(),
                                     _C._stream())
        assert status == 0, lib.mlk_last_error().decode()
        return out

    args = (x, in_w, x.new_empty(0), ln_w, ln_b, 1e-5, up_w, o_w, cos, sin, H, hd, nope, kvr, L, True, scale)
    packed = _C.mla_forward(*args)
    assert _C.mla_forward_launches() == ["mla_forward"]
    assert_bitwise(packed, row_major().cpu().numpy(), "packed vs row-major weights")
    with torch.no_grad():
        o_w.mul_(0.5)
        up_w.mul_(1.25)
    again = _C.mla_forward(*args)
    assert not torch.equal(again, packed), "the weight update must reach the kernel"
    assert_bitwise(again, row_major().cpu().numpy(), "packed vs row-major weights after an in-place update")
    # A `.data = new` swap keeps the object and its _version but moves data_ptr: the cache must see it.
    version = o_w._version
    o_w.data = (torch.randn(d, d, generator=g) * 0.05).to(dev, bf)
    assert o_w._version == version
    swapped = _C.mla_forward(*args)
    assert not torch.equal(swapped, again), "the swapped weight must reach the kernel"
    assert_bitwise(swapped, row_major().cpu().numpy(), "packed vs row-major weights after a .data swap")
    # On another stream the cached pack is reused (recorded on that stream) and gives the same bits.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        on_side = _C.mla_forward(*args)
    torch.cuda.current_stream().wait_stream(side)
    assert torch.equal(on_side, swapped)
    assert lib.mlk_mla_packed_elems(d, H, hd, nope, kvr) == _C.mla_pack_weights(in_w, up_w, o_w, H, hd, nope,
                                                                                 kvr).numel()
    assert lib.mlk_mla_packed_elems(d, H, hd, nope, 32) == 0, "no packed form without the per-window kernel"


def test_window_kernel_vs_oracle(dev, oracle):
    """The per-window kernel against the oracle chain at the MLA block geometry (bf16 weights: 2e-2)."""
    from montlok import _C

    rng = np.random.default_rng(31)
    B, L, d, H, hd, nope, kv_rank = 8, 128, 256, 8, 32, 16, 64
    x = rng.standard_normal((B, L, d)).astype(np.float32)
    p = _mla_params(rng, d, H, hd, nope, kv_rank, True)
    cos, sin = rope_tables(L, hd - nope)
    scale = 1.0 / math.sqrt(hd)

    def w(a):
        return _t(a, dev).to(torch.bfloat16)

    in_w = np.concatenate([p["q"], p["kv_down"], p["k_rope"]])
    out = _C.mla_forward(_t(x, dev), w(in_w), torch.empty(0, device=dev), _t(p["ln_w"], dev), _t(p["ln_b"], dev),
                         1e-5, w(p["kv_up"]), w(p["o"]), _t(cos, dev), _t(sin, dev), H, hd, nope, kv_rank, L, True,
                         scale)
    assert _C.mla_forward_launches() == ["mla_forward"]
    expect = _oracle_mla(oracle, x, p, H, hd, nope, kv_rank, L, True, scale, cos, sin)
    assert_close(out, expect, tol=BF16_TOL, name="per-window mla_forward vs oracle")


@pytest.mark.parametrize("scale", [-0.17677669529663687, 0.0])
def test_non_positive_scale_takes_the_scaled_softmax(dev, oracle, scale):
    """A softmax scale that is not positive: the per-window kernel declines (its max is taken over raw
    scores), the four-launch path runs the kernels' scaled-scores form, and the result still matches the
    oracle chain and the separate operators (their attention kernel in the same form) bit for bit."""
    from montlok import _C

    rng = np.random.default_rng(32)
    B, L, d, H, hd, nope, kv_rank = 4, 96, 256, 8, 32, 16, 64
    x = rng.standard_normal((B, L, d)).astype(np.float32)
    p = _mla_params(rng, d, H, hd, nope, kv_rank, True)
    cos, sin = rope_tables(L, hd - nope)

    def w(a):
        return _t(a, dev).to(torch.bfloat16)

    in_w = np.concatenate([p["q"], p["kv_down"], p["k_rope"]])
    args = (_t(x, dev), w(in_w), torch.empty(0, device=dev), _t(p["ln_w"], dev), _t(p["ln_b"], dev), 1e-5,
            w(p["kv_up"]), w(p["o"]), _t(cos, dev), _t(sin, dev), H, hd, nope, kv_rank, L, True, scale)
    out = _C._mla_forward(*args, allow_fused=True)
    assert _C.mla_forward_launches() == ["linear", "layer_norm_bf16", "mla_attend_normed", "linear"]
    separate = _C._mla_forward(*args, allow_fused=False)
    assert_bitwise(out, separate.cpu().numpy(), f"scale {scale}: fused attention vs separate operators")
    expect = _oracle_mla(oracle, x, p, H, hd, nope, kv_rank, L, True, scale, cos, sin)
    assert_close(out, expect, tol=BF16_TOL, name=f"scale {scale}: mla_forward vs oracle")


@pytest.mark.parametrize("geometry", sorted(MLA_GEOMETRIES))
def test_bf16_mla_vs_emulation(dev, oracle, geometry):
    """The bf16 MLA forms (the one-launch kernel where built, the four-launch path, the separate operators)
    against the float64 restatement of their roundings (tests/bf16_emu.py: normwise EMU_TOL, median row
    EMU_ROW_MEDIAN_TOL), and against the fp32 oracle chain within the 2e-2 contract; both printed."""
    from montlok import _C

    rng = np.random.default_rng(77)
    B, L, d, H, hd, nope, kvr = MLA_GEOMETRIES[geometry]
    x = rng.standard_normal((B, L, d)).astype(np.float32)
    p = _mla_params(rng, d, H, hd, nope, kvr, True)
    cos, sin = rope_tables(L, hd - nope)
    scale = 1.0 / math.sqrt(hd)
    bw = lambda a: _t(a, dev).to(torch.bfloat16)  # noqa: E731
    in_w = np.concatenate([p["q"], p["kv_down"], p["k_rope"]])
    args = (_t(x, dev), bw(in_w), torch.empty(0, device=dev), _t(p["ln_w"], dev), _t(p["ln_b"], dev), 1e-5,
            bw(p["kv_up"]), bw(p["o"]), _t(cos, dev), _t(sin, dev), H, hd, nope, kvr, L, True, scale)
    emulated = emu.mla_forward(x, p["q"], p["kv_down"], p["k_rope"], p["ln_w"], p["ln_b"], 1e-5, p["kv_up"], p["o"],
                               cos, sin, H, hd, nope, scale)
    fp32 = _oracle_mla(oracle, x, p, H, hd, nope, kvr, L, True, scale, cos, sin)
    paths = {"four launches": _C._mla_forward(*args, allow_fused=True, allow_window=False),
             "separate operators": _C._mla_forward(*args, allow_fused=False)}
    if geometry == "block":
        paths["one launch"] = _C._mla_forward(*args, allow_fused=True)
        assert _C.mla_forward_launches() == ["mla_forward"]
    for name, out in paths.items():
        e_orc = assert_close(out, fp32, tol=BF16_TOL, name=f"{geometry} {name} vs the fp32 oracle")
        m_orc = float(np.median(row_errors(out, fp32)))
        e_emu, m_emu = assert_emulated(out, emulated, name=f"{geometry} {name} vs the bf16 emulation")
        print(f"MLA {geometry} {name}: vs the bf16 emulation {e_emu:.2e} (median row {m_emu:.1e}), "
              f"vs the fp32 oracle {e_orc:.2e} (median row {m_orc:.1e})")


@pytest.mark.parametrize("B,Lq,Lk,H,hd,mask", ATTN_CASES)
def test_bf16_attention_vs_emulation(dev, oracle, B, Lq, Lk, H, hd, mask):
    """_C.attention in bf16 against the float64 restatement of its roundings (normwise EMU_TOL, median row
    EMU_ROW_MEDIAN_TOL); the fp32 oracle's distance printed beside it."""
    from montlok import _C

    rng = np.random.default_rng(B + Lq + Lk + hd + mask)
    q = rng.standard_normal((B, Lq, H, hd)).astype(np.float32)
    k = rng.standard_normal((B, Lk, H, hd)).astype(np.float32)
    v = rng.standard_normal((B, Lk, H, hd)).astype(np.float32)
    scale = 1.0 / math.sqrt(hd)
    out = _C.attention(_t(q, dev), _t(k, dev), _t(v, dev), mask, scale, torch.bfloat16)
    emulated = emu.attention(q, k, v, mask, scale)
    fp32 = oracle.sdpa(q, k, v, mask, scale)
    e_orc, m_orc = rel_err(out, fp32), float(np.median(row_errors(out, fp32)))
    e_emu, m_emu = assert_emulated(out, emulated, name="bf16 attention vs the emulation")
    print(f"bf16 attention {B}x{Lq}x{Lk} h{H} hd{hd} mask {mask}: vs the bf16 emulation {e_emu:.2e} "
          f"(median row {m_emu:.1e}), vs the fp32 oracle {e_orc:.2e} (median row {m_orc:.1e})")

"""GPU parity of the matrix-core linear and the ops built on it (linear,
swiglu_mlp, mamba3_siso_layer, stage1_forward).

The reference runs these GEMMs in oneDNN fp32 (montlok.cpp:67-91); the oracle
is an fp64 dot product rounded once. Gates (normwise relative error): fp32
weights 1e-5; bf16 weights 2e-2 against the fp32 product with the weights
upcast (the contract for bf16-weight configs), and 1e-6 against the exact
product of bf16-rounded inputs and weights, which pins what the kernel
computes: x rounded to bf16 (nearest even), fp32 accumulation.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import BF16_TOL, assert_close

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _bf16_round(a: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).bfloat16().float().numpy()


SHAPES = [(2048, 64, 304, False),    # RMSNorm->Mamba-3 block in_proj
          (2048, 128, 64, False),    # ... and out_proj
          (1000, 40, 256, True),     # raw-feature projection with bias
          (37, 7, 5, True),          # ragged everything
          (333, 300, 70, False),     # K beyond one 256-wide chunk
          (4100, 520, 1, True),      # one output column, two K chunks
          (1, 256, 336, False),      # a single row
          (64, 512, 1192, False),    # full-stack Mamba in_proj width
          (300, 96, 70, True),       # one wave per tile: ragged rows and N, K past the last 32-wide step
          (50, 200, 33, True),       # ... K = 200 (eight steps, the last two partly or wholly past K)
          (16, 8, 16, False),        # ... a single 8-wide k segment
          (9000, 256, 1192, True),   # bf16: the 32x32x16 form (wide output), ragged row block
          (5000, 96, 800, False)]    # ... K short of the chunk, N ragged


@pytest.mark.parametrize("M,K,N,with_bias", SHAPES)
def test_linear_fp32_weights(dev, oracle, M, K, N, with_bias):
    from montlok import _C

    rng = np.random.default_rng(M + K + N)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) if with_bias else None
    out = _C.linear(_t(x, dev), _t(w, dev), None if b is None else _t(b, dev))
    assert out.shape == (M, N)
    assert_close(out, oracle.linear(x, w, b), name=f"linear fp32 {M}x{K}->{N}")


@pytest.mark.parametrize("M,K,N,with_bias", SHAPES)
def test_linear_bf16_weights(dev, oracle, M, K, N, with_bias):
    from montlok import _C

    rng = np.random.default_rng(M * 3 + K + N)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = _bf16_round(rng.standard_normal((N, K)) * 0.02)
    b = rng.standard_normal(N).astype(np.float32) if with_bias else None
    out = _C.linear(_t(x, dev), _t(w, dev).bfloat16(), None if b is None else _t(b, dev))
    assert_close(out, oracle.linear(x, w, b), tol=BF16_TOL, name="bf16 weights vs fp32 product")
    assert_close(out, oracle.linear(_bf16_round(x), w, b), tol=1e-6, name="bf16 weights vs bf16-input product")


def test_linear_strided_input_and_leading_dims(dev, oracle):
    """A column slice of a wider buffer (montlok.cpp:52-55 accepts leading strides) and [B, L, K] inputs."""
    from montlok import _C

    rng = np.random.default_rng(5)
    wide = _t(rng.standard_normal((3, 50, 100)).astype(np.float32), dev)
    x = wide[:, :, 12:76]
    w = rng.standard_normal((48, 64)).astype(np.float32)
    out = _C.linear(x, _t(w, dev))
    assert out.shape == (3, 50, 48)
    assert_close(out, oracle.linear(x.cpu().numpy(), w), name="strided linear")


def test_linear_errors(dev):
    from montlok import _C

    x = torch.zeros(4, 8, device=dev)
    with pytest.raises(RuntimeError, match="input must end in in_features=16"):
        _C.linear(x, torch.zeros(3, 16, device=dev))
    with pytest.raises(RuntimeError, match="weight must be float32 or bfloat16"):
        _C.linear(x, torch.zeros(3, 8, device=dev, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="bias must have 3 elements"):
        _C.linear(x, torch.zeros(3, 8, device=dev), torch.zeros(4, device=dev))
    with pytest.raises(RuntimeError, match="input must be on the GPU"):
        _C.linear(torch.zeros(4, 8), torch.zeros(3, 8, device=dev))


def test_swiglu_mlp(dev, oracle):
    from montlok import _C

    rng = np.random.default_rng(21)
    x = rng.standard_normal((300, 64)).astype(np.float32)
    w_in = (rng.standard_normal((256, 64)) / 8).astype(np.float32)
    b_in = rng.standard_normal(256).astype(np.float32)
    w_out = (rng.standard_normal((64, 128)) / 11).astype(np.float32)
    out = _C.swiglu_mlp(_t(x, dev), _t(w_in, dev), _t(b_in, dev), _t(w_out, dev), None)
    expect = oracle.linear(oracle.swiglu(oracle.linear(x, w_in, b_in)), w_out)
    assert_close(out, expect, name="swiglu_mlp")


def _mamba_layer_params(rng, d_model, N, H, D, R, G=1):
    d_inner = H * D
    W = 2 * d_inner + 2 * G * N + 3 * H + R
    bound_in, bound_out = 1 / np.sqrt(d_model), 1 / np.sqrt(d_inner)
    return dict(in_w=rng.uniform(-bound_in, bound_in, (W, d_model)).astype(np.float32),
                out_w=rng.uniform(-bound_out, bound_out, (d_model, d_inner)).astype(np.float32),
                b_bias=np.ones((H, N), np.float32), c_bias=np.ones((H, N), np.float32),
                b_norm_w=np.ones(N, np.float32), c_norm_w=np.ones(N, np.float32),
                dt_bias=np.log(np.expm1(np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), H)))).astype(np.float32),
                skip=np.ones(H, np.float32))


_MAMBA_KEYS = ("in_w", "out_w", "b_bias", "c_bias", "b_norm_w", "c_norm_w", "dt_bias", "skip")


def _oracle_mamba_layer(oracle, x, p, N, G, H, D, R):
    projected = oracle.linear(x, p["in_w"])
    y = oracle.mamba3_siso_forward(projected, N, G, H, D, R, p["b_bias"], p["c_bias"], p["b_norm_w"], p["c_norm_w"],
                                   1e-5, 1e-5, p["dt_bias"], p["skip"], 1e-4)
    return oracle.linear(y, p["out_w"])


def test_mamba3_siso_layer_block_geometry(dev, oracle):
    """RMSNorm->Mamba-3 block: 64 windows x 32 tokens, d_model 64, 4 heads, d_state 16, expand 2."""
    from montlok import _C

    rng = np.random.default_rng(0)
    B, L, d, N, H, D, R = 64, 32, 64, 16, 4, 32, 4
    x = rng.standard_normal((B, L, d)).astype(np.float32)
    p = _mamba_layer_params(rng, d, N, H, D, R)
    out = _C.mamba3_siso_layer(_t(x, dev), *(_t(p[k], dev) for k in _MAMBA_KEYS), N, 1, H, D, R, 1e-5, 1e-5, 1e-4)
    assert_close(out, _oracle_mamba_layer(oracle, x, p, N, 1, H, D, R), name="mamba3_siso_layer")


def test_stage1_forward_two_layers(dev, oracle):
    """montlok.cpp:1011-1053 chained over two layers, against the same chain of oracle ops."""
    from montlok import _C

    rng = np.random.default_rng(3)
    B, L, d, N, H, D, R, groups = 4, 24, 64, 16, 4, 32, 4, 8
    x = rng.standard_normal((B, L, d)).astype(np.float32)
    packs_np = []
    for _ in range(2):
        p = _mamba_layer_params(rng, d, N, H, D, R)
        norm_w = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
        ffn_norm_w = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
        ffn_in = (rng.standard_normal((4 * d, d)) / 8).astype(np.float32)
        ffn_in_b = (0.1 * rng.standard_normal(4 * d)).astype(np.float32)
        ffn_out = (rng.standard_normal((d, 2 * d)) / 11).astype(np.float32)
        packs_np.append([norm_w] + [p[k] for k in _MAMBA_KEYS] + [ffn_norm_w, ffn_in, ffn_in_b, ffn_out,
                                                                   np.zeros(0, np.float32)])
    packs = [[_t(a, dev) for a in pack] for pack in packs_np]
    out = _C.stage1_forward(_t(x, dev), packs, 1e-5, groups, 1e-5, N, 1, H, D, R, 1e-5, 1e-5, 1e-4)

    hidden = x
    mamba_in = oracle.rms_norm(hidden, packs_np[0][0], 1e-5, groups)
    for i, pk in enumerate(packs_np):
        p = dict(zip(_MAMBA_KEYS, pk[1:9]))
        m = _oracle_mamba_layer(oracle, mamba_in, p, N, 1, H, D, R)
        hidden, normed = oracle.add_rms_norm(hidden, m, pk[9], 1e-5, 1)
        ffn = oracle.linear(oracle.swiglu(oracle.linear(normed, pk[10], pk[11])), pk[12])
        if i + 1 == len(packs_np):
            hidden = hidden + ffn
        else:
            hidden, mamba_in = oracle.add_rms_norm(hidden, ffn, packs_np[i + 1][0], 1e-5, groups)
    assert_close(out, hidden, name="stage1_forward")


# linear followed by the residual add, across the kernel forms: one wave per tile (small row
# counts), the row-layout form (fp32 weights, K within a chunk), the tiled form (bf16 weights,
# K within two chunks) and the K-chunked form (K beyond two chunks).
RESIDUAL_SHAPES = [(2048, 128, 64, False), (300, 96, 70, True), (20000, 128, 100, True), (9000, 256, 336, False),
                   (5000, 520, 40, True)]


@pytest.mark.parametrize("M,K,N,with_bias", RESIDUAL_SHAPES)
@pytest.mark.parametrize("wdt", ["f32", "bf16"])
def test_linear_residual_equals_linear_then_add(dev, M, K, N, with_bias, wdt):
    from montlok import _C

    g = torch.Generator(device="cpu").manual_seed(M + K + N)
    x = torch.randn(M, K, generator=g).to(dev)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(dev)
    if wdt == "bf16":
        w = w.bfloat16()
    b = torch.randn(N, generator=g).to(dev) if with_bias else None
    r = torch.randn(M, N, generator=g).to(dev)
    fused = _C.linear_residual(x, w, b, r)
    separate = r + _C.linear(x, w, b)
    assert torch.equal(fused, separate), f"{M}x{K}->{N} {wdt}"


@pytest.mark.parametrize("M,K,N,groups", [(2048, 64, 304, 8), (300, 64, 70, 4), (1000, 128, 96, 2), (77, 128, 33, 8),
                                          (500, 256, 64, 4), (64, 256, 300, 16), (250, 96, 50, 12),
                                          (300, 128, 40, 4)])
@pytest.mark.parametrize("wdt", ["f32", "bf16"])
def test_rms_norm_linear_equals_the_two_operators(dev, M, K, N, groups, wdt):
    """Groups of 8, 16, 32 and 64 floats on the fused form, bit for bit against rms_norm then linear."""
    from montlok import _C

    g = torch.Generator(device="cpu").manual_seed(M * 7 + K + N + groups)
    x = (torch.randn(M, K, generator=g) * 3).to(dev)
    nw = (torch.rand(K, generator=g) + 0.5).to(dev)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(dev)
    if wdt == "bf16":
        w = w.bfloat16()
    b = torch.randn(N, generator=g).to(dev)
    fused = _C.rms_norm_linear(x, nw, 1e-5, groups, w, b)
    separate = _C.linear(_C.rms_norm(x, nw, 1e-5, groups), w, b)
    assert torch.equal(fused, separate), f"{M}x{K}->{N} groups {groups} {wdt}"


@pytest.mark.parametrize("M,N,groups", [(65536, 668, 8), (40000, 257, 16), (4097, 64, 4), (9000, 100, 2)])
def test_rms_norm_linear_large_rows(dev, M, N, groups):
    """fp32 weights with in_features 128 take the row-layout form at any row count (the streaming decode's
    GroupedRMSNorm + in_proj): one launch, bit for bit against rms_norm then linear."""
    from montlok import _C
    from montlok._C import _load

    K = 128
    g = torch.Generator(device="cpu").manual_seed(M + N + groups)
    x = (torch.randn(M, K, generator=g) * 3).to(dev)
    nw = (torch.rand(K, generator=g) + 0.5).to(dev)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(dev)
    b = torch.randn(N, generator=g).to(dev)
    out = torch.empty(M, N, device=dev)
    status = _load().mlk_rms_norm_linear(x.data_ptr(), M, K, K, nw.data_ptr(), 1e-5, groups, w.data_ptr(), 0,
                                         b.data_ptr(), N, out.data_ptr(), N, torch.cuda.current_stream().cuda_stream)
    assert status == 0, "the shape has the fused form"
    separate = _C.linear(_C.rms_norm(x, nw, 1e-5, groups), w, b)
    assert torch.equal(out, separate), f"{M}x{K}->{N} groups {groups}"


def test_rms_norm_linear_beyond_the_fused_form(dev):
    """Row counts that fill the chip, and groups of 4 floats, run the two operators."""
    from montlok import _C
    from montlok._C import _load

    g = torch.Generator(device="cpu").manual_seed(9)
    for M, K, groups in ((40000, 64, 8), (100, 64, 16)):
        x = torch.randn(M, K, generator=g).to(dev)
        nw = (torch.rand(K, generator=g) + 0.5).to(dev)
        w = (torch.randn(48, K, generator=g) / 8).to(dev)
        out = torch.empty(M, 48, device=dev)
        status = _load().mlk_rms_norm_linear(x.data_ptr(), M, K, K, nw.data_ptr(), 1e-5, groups, w.data_ptr(), 0, None,
                                             48, out.data_ptr(), 48, torch.cuda.current_stream().cuda_stream)
        assert status == 3
        fused = _C.rms_norm_linear(x, nw, 1e-5, groups, w)
        assert torch.equal(fused, _C.linear(_C.rms_norm(x, nw, 1e-5, groups), w))


def test_streaming_forms_full_size(dev, monkeypatch):
    """The stack's Mamba in_proj at its full size, 262144 x 256 -> 1192 (bf16 weights): the IO-wave form,
    the storing-wave form, the plain streaming form and linear_t32_kernel give the same bits (a property
    that holds at any size; the oracle comparisons above run at sizes the CPU finishes quickly)."""
    from montlok import _C

    g = torch.Generator().manual_seed(1192)
    x = torch.randn(262144, 256, generator=g).to(dev)
    w = (torch.randn(1192, 256, generator=g) * 0.02).to(dev).bfloat16()
    outs = {}
    for form, env in (("io", {}), ("sw", {"MLK_LINEAR_STORE_WAVES": "sw"}), ("plain", {"MLK_LINEAR_STORE_WAVES": "0"}),
                      ("t32", {"MLK_LINEAR_FORM": "t32"})):
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        outs[form] = _C.linear(x, w)
        for k in env:
            monkeypatch.delenv(k)
    assert torch.isfinite(outs["io"]).all().item()
    for form in ("sw", "plain", "t32"):
        assert torch.equal(outs["io"], outs[form]), f"IO-wave form vs {form}"


@pytest.mark.parametrize("M,N,bias,strided", [(40000, 256, False, False), (33000, 192, True, True), (35000, 320, True, False)])
def test_streaming_form_k512(dev, oracle, M, N, bias, strided, monkeypatch):
    """bf16 weights, K = 512, 128 or more output columns, 32768 or more rows: the streaming form with the W
    fragments of all of K in registers (ragged column groups, strided x, bias, the residual epilogue)
    matches the exact product of bf16-rounded inputs at 1e-6, and the tiled 16 x 16 x 32 form
    (MLK_LINEAR_FORM=t32) to the same bound (their k blockings differ, so not bit for bit)."""
    from montlok import _C

    rng = np.random.default_rng(M + N + 512)
    K = 512
    xw = rng.standard_normal((M, K + (16 if strided else 0))).astype(np.float32)
    x = _t(xw, dev)[:, 8:8 + K] if strided else _t(xw, dev)
    w = _bf16_round(rng.standard_normal((N, K)) * 0.02)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    args = (x, _t(w, dev).bfloat16(), None if b is None else _t(b, dev))
    res = torch.randn(M, N, generator=torch.Generator().manual_seed(M)).to(dev)
    streaming = _C.linear(*args)
    with_res = _C.linear_residual(*args, res)
    monkeypatch.setenv("MLK_LINEAR_FORM", "t32")
    tiled = _C.linear(*args)
    monkeypatch.delenv("MLK_LINEAR_FORM")
    assert torch.equal(with_res, res + streaming), "residual epilogue vs the two steps"
    x_np = xw[:, 8:8 + K] if strided else xw
    expect = oracle.linear(_bf16_round(x_np), w, b)
    assert_close(streaming, expect, tol=1e-6, name="K=512 streaming vs bf16-input product")
    assert_close(tiled, expect, tol=1e-6, name="K=512 tiled vs bf16-input product")


@pytest.mark.parametrize("M,N,bias,strided", [(9000, 1192, True, False), (70000, 1192, False, True), (31, 768, True, False),
                                              (4096, 2000, False, False), (50001, 1196, True, True),
                                              (20000, 1194, False, False), (1500, 1192, False, True)])
def test_streaming_form_equals_t32_form(dev, oracle, M, N, bias, strided, monkeypatch):
    """bf16 weights, K = 256, 12 or more 64-column chunks: the streaming forms (weights in registers, x
    tiles through LDS; by default the form with IO waves where the output allows it (no residual,
    N % 4 = 0; N = 1194 and the residual calls take the next form), MLK_LINEAR_STORE_WAVES=sw the form
    with storing waves, =0 the one with neither) give linear_t32_kernel's result bit for bit
    (MLK_LINEAR_FORM=t32 selects that form), also with the residual epilogue, at row counts that leave
    blocks without a tile (31, 1500 rows) or a ragged last tile, and all match the product of bf16-rounded
    inputs."""
    from montlok import _C

    rng = np.random.default_rng(M + N)
    K = 256
    xw = rng.standard_normal((M, K + (16 if strided else 0))).astype(np.float32)
    x = _t(xw, dev)[:, 8:8 + K] if strided else _t(xw, dev)
    w = _bf16_round(rng.standard_normal((N, K)) * 0.02)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    args = (x, _t(w, dev).bfloat16(), None if b is None else _t(b, dev))
    res = torch.randn(M, N, generator=torch.Generator().manual_seed(M)).to(dev)

    def both():
        return _C.linear(*args), _C.linear_residual(*args, res)

    streaming = both()
    monkeypatch.setenv("MLK_LINEAR_STORE_WAVES", "sw")
    store_waves = both()
    monkeypatch.setenv("MLK_LINEAR_STORE_WAVES", "0")
    in_wave = both()
    monkeypatch.setenv("MLK_LINEAR_FORM", "t32")
    t32 = both()
    monkeypatch.delenv("MLK_LINEAR_FORM")
    monkeypatch.delenv("MLK_LINEAR_STORE_WAVES")
    for name, a, c in (("streaming", streaming, t32), ("streaming, storing waves", store_waves, t32),
                       ("streaming, stores on the computing waves", in_wave, t32)):
        assert torch.equal(a[0], c[0]), f"{name} vs linear_t32_kernel"
        assert torch.equal(a[1], c[1]), f"{name} with residual vs linear_t32_kernel"
    assert torch.equal(streaming[1], res + streaming[0]), "residual epilogue vs the two steps"
    x_np = xw[:, 8:8 + K] if strided else xw
    assert_close(streaming[0], oracle.linear(_bf16_round(x_np), w, b), tol=1e-6, name="bf16-input product")

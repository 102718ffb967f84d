"""GPU parity of the row-wise layers (RMSNorm, add+RMSNorm, LayerNorm, SwiGLU).

Each HIP kernel is called through the C ABI (montlok._C -> libmlk_hip.so) and
compared with the golden vectors of the compiled reference and with the CPU
oracle on the same seeded inputs. Gate: normwise relative error <= 1e-5
(fp32); the number of elements that differ bitwise is reported.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close, bit_mismatches

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_rms_norm_golden(dev, golden):
    from montlok import _C

    g = golden("norms")
    for i in range(4):
        groups, eps = g[f"rms{i}_meta"]
        x, w = _t(g[f"rms{i}_x"], dev), _t(g[f"rms{i}_w"], dev)
        out = _C.rms_norm(x, w, float(eps), int(groups))
        assert_close(out, g[f"rms{i}_out"], name=f"rms{i}")
        res, nrm = _C.add_rms_norm(x, _t(g[f"rms{i}_right"], dev), w, float(eps), int(groups))
        assert bit_mismatches(res, g[f"rms{i}_residual"]) == 0
        assert_close(nrm, g[f"rms{i}_normalized"], name=f"add_rms{i}")


def test_layer_norm_and_swiglu_golden(dev, golden):
    from montlok import _C

    g = golden("norms")
    for i in range(3):
        b = g.get(f"ln{i}_b")
        out = _C.layer_norm(_t(g[f"ln{i}_x"], dev), _t(g[f"ln{i}_w"], dev), None if b is None else _t(b, dev), 1e-5)
        assert_close(out, g[f"ln{i}_out"], name=f"ln{i}")
    for i in range(2):
        assert_close(_C.swiglu(_t(g[f"swiglu{i}_x"], dev)), g[f"swiglu{i}_out"], name=f"swiglu{i}")


@pytest.mark.parametrize("rows,dim,groups", [(2048, 64, 8), (4096, 256, 1), (1000, 128, 1), (333, 512, 1),
                                             (64, 1024, 2), (77, 100, 4), (5, 12, 3)])
def test_rms_norm_vs_oracle(dev, oracle, rows, dim, groups):
    from montlok import _C

    rng = np.random.default_rng(rows + dim)
    x = (rng.standard_normal((rows, dim)) * 3).astype(np.float32)
    w = (rng.random(dim) + 0.5).astype(np.float32)
    out = _C.rms_norm(_t(x, dev), _t(w, dev), 1e-5, groups)
    expect = oracle.rms_norm(x, w, 1e-5, groups)
    assert_close(out, expect, name="rms_norm")
    # Squares of fp32 values are exact in double: bitwise agreement expected.
    assert bit_mismatches(out, expect) <= max(1, x.size // 10000)


@pytest.mark.parametrize("rows,dim,groups", [(262147, 256, 1), (65541, 64, 1), (140003, 64, 8), (20001, 1024, 1)])
def test_norms_four_rows_per_lane_group(dev, oracle, rows, dim, groups):
    """Launches of 4096 blocks or more give each lane group four rows (every row's loads issued before
    the first reduction): rms_norm and add_rms_norm at the stack's 262,144 x 256 (plus a ragged tail of
    rows), grouped, and wide rows, against the oracle; the residual of add_rms_norm bit for bit (one fp32
    add), the normalised rows as the single-row kernels are (fp64 sums, one rounding)."""
    from montlok import _C

    rng = np.random.default_rng(rows + dim + groups)
    x = (rng.standard_normal((rows, dim)) * 3).astype(np.float32)
    r = rng.standard_normal((rows, dim)).astype(np.float32)
    w = (rng.random(dim) + 0.5).astype(np.float32)
    tx, tw = _t(x, dev), _t(w, dev)
    out = _C.rms_norm(tx, tw, 1e-5, groups)
    expect = oracle.rms_norm(x, w, 1e-5, groups)
    assert_close(out, expect, name="rms_norm")
    assert bit_mismatches(out, expect) <= max(1, x.size // 10000)
    res, nrm = _C.add_rms_norm(tx, _t(r, dev), tw, 1e-5, groups)
    e_res, e_nrm = oracle.add_rms_norm(x, r, w, 1e-5, groups)
    assert bit_mismatches(res, e_res) == 0, "residual"
    assert_close(nrm, e_nrm, name="add_rms_norm")
    assert bit_mismatches(nrm, e_nrm) <= max(1, x.size // 10000)
    if groups == 1 and dim <= 256:
        b = rng.standard_normal(dim).astype(np.float32)
        assert_close(_C.layer_norm(tx, tw, _t(b, dev), 1e-5), oracle.layer_norm(x, w, b, 1e-5), name="layer_norm")


def test_rms_norm_strided_rows(dev, oracle):
    from montlok import _C

    rng = np.random.default_rng(3)
    base = rng.standard_normal((64, 37)).astype(np.float32)
    w = (rng.random(64) + 0.5).astype(np.float32)
    x = _t(base, dev).t()  # [37, 64] with a non-unit last stride: copied dense like the reference
    out = _C.rms_norm(x, _t(w, dev), 1e-6, 1)
    assert_close(out, oracle.rms_norm(base.T, w, 1e-6, 1))
    wide = _t(rng.standard_normal((37, 96)).astype(np.float32), dev)
    view = wide[:, 8:72]  # row stride 96, dense last dim
    assert_close(_C.rms_norm(view, _t(w, dev), 1e-6, 2), oracle.rms_norm(view.cpu().numpy(), w, 1e-6, 2))


@pytest.mark.parametrize("rows,dim,bias", [(32768, 64, True), (1000, 256, False), (37, 66, True), (3, 1, True)])
def test_layer_norm_vs_oracle(dev, oracle, rows, dim, bias):
    from montlok import _C

    rng = np.random.default_rng(dim)
    x = (rng.standard_normal((rows, dim)) * 2 + 0.5).astype(np.float32)
    w = (rng.random(dim) + 0.5).astype(np.float32)
    b = rng.standard_normal(dim).astype(np.float32) if bias else None
    out = _C.layer_norm(_t(x, dev), _t(w, dev), None if b is None else _t(b, dev), 1e-5)
    assert_close(out, oracle.layer_norm(x, w, b, 1e-5), name="layer_norm")


def test_layer_norm_strided_latent_slice(dev, oracle):
    """kv_latent is a column slice of the fused projection (montlok.cpp:1190-1193)."""
    from montlok import _C

    rng = np.random.default_rng(4)
    proj = rng.standard_normal((4, 33, 336)).astype(np.float32)
    w = (rng.random(64) + 0.5).astype(np.float32)
    b = rng.standard_normal(64).astype(np.float32)
    t = _t(proj, dev)
    out = _C.layer_norm(t[..., 256:320], _t(w, dev), _t(b, dev), 1e-5)
    assert_close(out, oracle.layer_norm(proj[..., 256:320], w, b, 1e-5))


def test_swiglu_vs_oracle(dev, oracle):
    from montlok import _C

    rng = np.random.default_rng(5)
    x = (rng.standard_normal((4097, 2 * 384)) * 3).astype(np.float32)
    assert_close(_C.swiglu(_t(x, dev)), oracle.swiglu(x))


def test_layer_errors(dev):
    from montlok import _C

    x = torch.zeros(4, 10, device=dev)
    with pytest.raises(RuntimeError, match="groups must divide"):
        _C.rms_norm(x, torch.ones(10, device=dev), 1e-5, 3)
    with pytest.raises(RuntimeError, match="weight must have 10 elements"):
        _C.rms_norm(x, torch.ones(9, device=dev), 1e-5, 1)
    with pytest.raises(RuntimeError, match="x must be on the GPU"):
        _C.rms_norm(x.cpu(), torch.ones(10, device=dev), 1e-5, 1)
    with pytest.raises(RuntimeError, match="x must be float32"):
        _C.layer_norm(x.double(), torch.ones(10, device=dev), None, 1e-5)
    with pytest.raises(RuntimeError, match="even dimension"):
        _C.swiglu(torch.zeros(3, 5, device=dev))

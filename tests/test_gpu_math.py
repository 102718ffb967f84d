"""Error bounds of the kernels' double-precision device math (exp, tanh,
sigmoid, reciprocal) against numpy's correctly rounded-in-practice libm, in
the spirit of the reference self-test of its own exp (<= 4 double ulp,
rdt4quant_cpu/montlok_selftest.cpp:789-790)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ulp_err(got, expect):
    got = np.asarray(got, dtype=np.float64)
    expect = np.asarray(expect, dtype=np.float64)
    spacing = np.spacing(np.abs(expect))
    spacing[spacing == 0] = np.finfo(np.float64).tiny
    return np.abs(got - expect) / spacing


def test_device_math_bounds(dev):
    from montlok import _C

    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-40, 40, 200000), rng.uniform(-1e-3, 1e-3, 20000),
                        np.array([0.0, -0.0, 1.0, -1.0, 700.0, -700.0, 709.7, -745.0])])
    out = {k: v.cpu().numpy() for k, v in _C.math_check(torch.from_numpy(x).to(dev)).items()}
    assert _ulp_err(out["exp"], np.exp(x)).max() <= 4
    # tanh: absolute error (the kernels add it to an O(1) bias).
    assert np.abs(out["tanh"] - np.tanh(x)).max() <= 4e-16
    with np.errstate(over="ignore"):  # exp(745) is inf in numpy too: the reference sigmoid is then 0
        assert np.abs(out["sigmoid"] - 1 / (1 + np.exp(-x))).max() <= 4e-16
    pos = np.abs(x) + 0.5
    r = _C.math_check(torch.from_numpy(pos).to(dev))["recip"].cpu().numpy()
    assert _ulp_err(r, 1.0 / pos).max() <= 1
    # After rounding to float32 exp agrees with the correctly rounded value.
    sel = np.abs(x) < 80
    assert np.mean(out["exp"][sel].astype(np.float32) != np.exp(x[sel]).astype(np.float32)) < 1e-5
    # Special values (the last eight inputs): 0, -0, 1, -1, 700, -700, 709.7, -745.
    sp = {k: v[-8:] for k, v in out.items()}
    assert sp["tanh"][0] == 0.0 and sp["tanh"][1] == 0.0 and np.signbit(sp["tanh"][1])
    assert abs(sp["tanh"][2] - np.tanh(1.0)) < 4e-16 and abs(sp["tanh"][3] + np.tanh(1.0)) < 4e-16
    assert sp["exp"][0] == 1.0 and np.isfinite(sp["exp"][6]) and sp["exp"][6] > 1e308
    assert _ulp_err(sp["exp"][4:6], np.exp(np.array([700.0, -700.0]))).max() <= 4

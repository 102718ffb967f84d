"""The reference's A/B switches on the GPU path (README.md:265-280,
python/montlok/rdt/mamba3.py:50-54, model.py:47-55, 144-148): each one changes
the path a module takes, and the result stays within the tolerance the
reference's own tests give that pair.

- MONTLOK_CPP_FUSED=0: Mamba-3 pre-processing as tensor operations + the
  recurrence kernel alone, against the fused layer and against the oracle at
  2e-5 (1 + max|y|) (tests/rdt/test_rdt_kernels.py:126-128).
- MONTLOK_CPP_TAIL=0, MONTLOK_CPP_NATIVE_STAGE1=0, MONTLOK_CPP_NATIVE_STAGE2=0:
  the model's quantiles against the default path at 1e-5 normwise.
- MONTLOK_CPP_MHC=0, MONTLOK_CPP_LAYERS=0, MONTLOK_CPP=0: the reference runs
  upstream PyTorch there; this package has no such forward and raises.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close, to_np
from test_gpu_model import _model
from test_gpu_modules import _mamba_oracle

pytestmark = pytest.mark.gpu

_SWITCHES = ("MONTLOK_CPP_FUSED", "MONTLOK_CPP_TAIL", "MONTLOK_CPP_NATIVE_STAGE1", "MONTLOK_CPP_NATIVE_STAGE2",
             "MONTLOK_CPP_MHC", "MONTLOK_CPP_LAYERS")


@pytest.fixture
def clean_env(monkeypatch):
    monkeypatch.setenv("MONTLOK_CPP", "1")
    for name in _SWITCHES:
        monkeypatch.delenv(name, raising=False)
    return monkeypatch


def _assert_ref_tol(actual, expected, tol, name):
    a, e = to_np(actual).astype(np.float64), np.asarray(to_np(expected), dtype=np.float64)
    assert np.isfinite(a).all(), name
    diff = np.abs(a - e).max()
    bound = tol * (1.0 + np.abs(e).max())
    assert diff <= bound, f"{name}: max|diff| {diff:.3e} > {bound:.3e}"


@pytest.mark.parametrize("d_model,d_state,headdim,ngroups,B,L", [(64, 16, 16, 1, 2, 48), (48, 14, 8, 2, 2, 37),
                                                                  (64, 16, 32, 1, 3, 20), (256, 64, 64, 1, 1, 96)])
def test_fused_off_runs_the_recurrence_kernel(dev, oracle, clean_env, d_model, d_state, headdim, ngroups, B, L):
    from montlok.rdt import Mamba3HIP
    from montlok.rdt.mamba3 import cpp_backend

    torch.manual_seed(7)
    m = Mamba3HIP(d_model, d_state=d_state, expand=2, headdim=headdim, ngroups=ngroups).eval()
    with torch.no_grad():
        m.B_bias.add_(torch.randn_like(m.B_bias) * 0.3)
        m.C_bias.add_(torch.randn_like(m.C_bias) * 0.3)
        m.B_norm.weight.mul_(torch.rand_like(m.B_norm.weight) + 0.5)
        m.C_norm.weight.mul_(torch.rand_like(m.C_norm.weight) + 0.5)
        m.D.add_(torch.randn_like(m.D) * 0.5)
        m.dt_bias.add_(torch.randn_like(m.dt_bias) * 0.5)
    x = torch.randn(B, L, d_model)
    expect = _mamba_oracle(oracle, m, x.numpy())
    m = m.to(dev)
    with torch.no_grad():
        assert cpp_backend() == "fused"
        fused = m(x.to(dev))
        clean_env.setenv("MONTLOK_CPP_FUSED", "0")
        assert cpp_backend() == "recurrent"
        recurrent = m(x.to(dev))
    _assert_ref_tol(recurrent, expect, 2e-5, "FUSED=0 vs oracle")
    _assert_ref_tol(recurrent, fused.cpu(), 2e-5, "FUSED=0 vs fused")
    assert not torch.equal(recurrent, fused), "the switch must change the path"


@pytest.mark.parametrize("switch", ["MONTLOK_CPP_TAIL", "MONTLOK_CPP_NATIVE_STAGE1", "MONTLOK_CPP_NATIVE_STAGE2",
                                    "MONTLOK_CPP_FUSED"])
def test_model_switches_keep_the_result(dev, clean_env, switch):
    from montlok.rdt import model as model_mod

    m = _model(seed=9).to(dev)
    x = torch.randn(2, 24, 7, generator=torch.Generator().manual_seed(9)).to(dev)
    with torch.no_grad():
        base, _ = m(x, 2)
        clean_env.setenv(switch, "0")
        flags = (model_mod.tail_enabled(), model_mod.native_stage1_enabled(), model_mod.native_stage2_enabled())
        other, _ = m(x, 2)
    expect_off = {"MONTLOK_CPP_TAIL": 0, "MONTLOK_CPP_NATIVE_STAGE1": 1, "MONTLOK_CPP_NATIVE_STAGE2": 2,
                  "MONTLOK_CPP_FUSED": 1}[switch]
    assert not flags[expect_off], f"{switch}=0 must switch its path off"
    tol = 2e-5 if switch == "MONTLOK_CPP_FUSED" else 1e-5
    assert_close(other, base, tol=tol, name=f"{switch}=0 vs default")


@pytest.mark.parametrize("switch", ["MONTLOK_CPP_MHC", "MONTLOK_CPP_LAYERS"])
def test_family_switches_raise(dev, clean_env, switch):
    from montlok.rdt import ManifoldHyperConnectionHIP, RMSNormHIP

    module = ManifoldHyperConnectionHIP(16, n_streams=2).to(dev) if switch == "MONTLOK_CPP_MHC" else \
        RMSNormHIP(16).to(dev)
    x = torch.randn(1, 3, 2, 16, device=dev) if switch == "MONTLOK_CPP_MHC" else torch.randn(3, 16, device=dev)
    clean_env.setenv(switch, "0")
    with torch.no_grad(), pytest.raises(RuntimeError, match="switched off"):
        module(x, lambda a: a) if switch == "MONTLOK_CPP_MHC" else module(x)

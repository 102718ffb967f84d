"""The reference's A/B switches on the GPU path (README.md:265-280,
python/montlok/rdt/mamba3.py:50-54, model.py:47-55, 144-148): each one changes
the path a module takes, and the result stays within the tolerance the
reference's own tests give that pair.

- MONTLOK_CPP_FUSED=0: Mamba-3 pre-processing as tensor operations + the
  recurrence kernel alone, against the fused layer and against the oracle at
  2e-5 (1 + max|y|) (tests/rdt/test_rdt_kernels.py:126-128).
- MONTLOK_CPP_TAIL=0, MONTLOK_CPP_NATIVE_STAGE1=0, MONTLOK_CPP_NATIVE_STAGE2=0:
  the model's quantiles against the default path at 1e-5 normwise.
- MONTLOK_CPP_MHC=0, MONTLOK_CPP_LAYERS=0, MONTLOK_CPP=0: the upstream
  PyTorch forward of that family on the device (no kernel called), against the
  kernel path at 2e-5 (1 + max|y|).
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


def _no_kernels(monkeypatch, *modules):
    """Make every kernel call of the given drop-in modules fail, so a result proves the PyTorch path ran."""

    def refuse():
        raise AssertionError("a kernel was called with its family switched off")

    for mod in modules:
        monkeypatch.setattr(mod, "ext", refuse)


@pytest.mark.parametrize("switch", ["MONTLOK_CPP_MHC", "MONTLOK_CPP_LAYERS", "MONTLOK_CPP"])
def test_family_switches_run_upstream_pytorch(dev, clean_env, switch):
    """Each family switch runs that family's upstream PyTorch forward on the device (no kernel is called),
    within the reference's PyTorch-vs-kernel tolerance 2e-5 (1 + max|y|) of the kernel path."""
    import montlok.rdt.layers as layers_mod
    import montlok.rdt.mamba3 as mamba_mod
    import montlok.rdt.mhc as mhc_mod
    import montlok.rdt.mla as mla_mod
    from types import SimpleNamespace

    from montlok.rdt import MLAHIP, ManifoldHyperConnectionHIP, Mamba3HIP, RMSNormHIP

    torch.manual_seed(9)
    hc = ManifoldHyperConnectionHIP(64, n_streams=4).to(dev)
    with torch.no_grad():
        for a in (hc.pre_alpha, hc.post_alpha, hc.res_alpha):
            a.fill_(0.7)
        hc.res_bias.normal_()
    norm = RMSNormHIP(64).to(dev)
    cfg = SimpleNamespace(d_model=64, n_heads=2, head_dim=32, nope_head_dim=16, rope_head_dim=16, kv_lora_rank=32,
                          q_lora_rank=0, rope_theta=10000.0)
    mla = MLAHIP(cfg).to(dev).eval()
    mamba = Mamba3HIP(64, d_state=16, headdim=32).to(dev).eval()
    streams = torch.randn(2, 20, 4, 64, device=dev)

    def run():
        with torch.no_grad():
            return (hc(streams, lambda agg: mla(norm(agg))), mamba(norm(streams[:, :, 0])))

    kernels = run()
    clean_env.setenv(switch, "0")
    families = {"MONTLOK_CPP_MHC": (mhc_mod,), "MONTLOK_CPP_LAYERS": (layers_mod, mla_mod),
                "MONTLOK_CPP": (mhc_mod, layers_mod, mla_mod, mamba_mod)}[switch]
    _no_kernels(clean_env, *families)
    upstream = run()
    for name, a, b in zip(("mHC over RMSNorm -> MLA", "RMSNorm -> Mamba-3"), upstream, kernels):
        _assert_ref_tol(a, b, 2e-5, f"{switch}=0: {name}")


def test_model_with_kernels_off(dev, clean_env):
    """MONTLOK_CPP=0: the model runs the upstream module chain on the device; its quantiles agree with the
    kernel path within the reference's tolerance for a PyTorch-vs-kernel pair."""
    import montlok.rdt.layers as layers_mod
    import montlok.rdt.mamba3 as mamba_mod
    import montlok.rdt.mhc as mhc_mod
    import montlok.rdt.mla as mla_mod
    import montlok.rdt.model as model_mod

    m = _model(seed=4).to(dev)
    x = torch.randn(2, 24, 7, generator=torch.Generator().manual_seed(4)).to(dev)
    with torch.no_grad():
        base, _ = m(x, 2)
    clean_env.setenv("MONTLOK_CPP", "0")
    _no_kernels(clean_env, layers_mod, mamba_mod, mhc_mod, mla_mod, model_mod)
    with torch.no_grad():
        other, _ = m(x, 2)
    _assert_ref_tol(other, base, 2e-5, "MONTLOK_CPP=0 model")

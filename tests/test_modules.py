"""Drop-in modules without a GPU: the parameter contract of the reference's
modules (state-dict names and shapes) and the refusal to run anywhere but the
GPU path."""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch
from torch import nn


def test_mamba3_parameter_contract():
    """python/montlok/rdt/mamba3.py:109-141: names, shapes and the rotary-angle rule."""
    from montlok.rdt import Mamba3CPUReference, Mamba3HIP

    assert Mamba3CPUReference is Mamba3HIP
    m = Mamba3HIP(64, d_state=16, expand=2, headdim=32)
    shapes = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    assert shapes == {"in_proj.weight": (304, 64), "dt_bias": (4,), "B_bias": (4, 1, 16), "C_bias": (4, 1, 16),
                      "B_norm.weight": (16,), "C_norm.weight": (16,), "D": (4,), "out_proj.weight": (64, 128)}
    assert m.num_rope_angles == 4
    assert Mamba3HIP(128, d_state=64, headdim=64).num_rope_angles == 16
    assert Mamba3HIP(64, d_state=14, headdim=32, rope_fraction=0.5).num_rope_angles == 3
    dt = torch.nn.functional.softplus(m.dt_bias)
    assert bool(((dt >= 1e-4 * 0.999) & (dt <= 0.1 * 1.001)).all())


def test_mhc_parameter_contract_and_init():
    """reference/Model/layers/mhc.py:118-150: sigmoid(pre) = 1/n, 2 sigmoid(post) = 1, res bias 3 I."""
    from montlok.rdt import ManifoldHyperConnectionCPU, ManifoldHyperConnectionHIP

    assert ManifoldHyperConnectionCPU is ManifoldHyperConnectionHIP
    h = ManifoldHyperConnectionHIP(128, n_streams=4)
    shapes = {k: tuple(v.shape) for k, v in h.state_dict().items()}
    assert shapes == {"pre_bias": (4,), "post_bias": (4,), "res_bias": (4, 4), "dyn_norm.weight": (128,),
                      "pre_proj.weight": (4, 128), "post_proj.weight": (4, 128), "res_proj.weight": (16, 128),
                      "pre_alpha": (), "post_alpha": (), "res_alpha": ()}
    assert torch.allclose(torch.sigmoid(h.pre_bias), torch.full((4,), 0.25))
    assert torch.equal(h.res_bias, torch.eye(4) * 3)
    w = h._projection_block()
    assert w.dtype == torch.float64 and w.shape == (24, 128)
    assert w is h._projection_block()  # cached
    with torch.no_grad():
        h.pre_proj.weight.add_(1.0)  # bumps the version: the cache is rebuilt
    assert w is not h._projection_block()


def test_mla_parameter_contract():
    """reference/Model/layers/mla.py:43-67 (q_lora_rank 0 and > 0)."""
    from montlok.rdt import MLACPU, MLAHIP

    assert MLACPU is MLAHIP
    cfg = SimpleNamespace(d_model=256, n_heads=8, head_dim=32, nope_head_dim=16, rope_head_dim=16, kv_lora_rank=64,
                          q_lora_rank=0, rope_theta=10000.0)
    shapes = {k: tuple(v.shape) for k, v in MLAHIP(cfg).state_dict().items()}
    assert shapes == {"q_proj.weight": (256, 256), "kv_down.weight": (64, 256), "kv_norm.weight": (64,),
                      "kv_norm.bias": (64,), "kv_up.weight": (384, 64), "k_rope_proj.weight": (16, 256),
                      "o_proj.weight": (256, 256)}
    cfg.q_lora_rank = 32
    keys = set(MLAHIP(cfg).state_dict())
    assert {"q_down.weight", "q_norm.weight", "q_norm.bias", "q_up.weight"} <= keys and "q_proj.weight" not in keys
    cfg.head_dim = 40
    with pytest.raises(ValueError, match="head_dim must equal"):
        MLAHIP(cfg)


def test_layers_install_and_contract():
    from montlok.rdt import GroupedRMSNormCPU, LayerNormCPU, RMSNormCPU, SwiGLUCPU, install_cpu_layers

    class RMSNorm(nn.Module):  # stands for the upstream class of the same name and attributes
        def __init__(self):
            super().__init__()
            self.dim, self.eps = 8, 1e-5
            self.weight = nn.Parameter(torch.ones(8))

    model = nn.Sequential(RMSNorm(), nn.LayerNorm(8), nn.Linear(8, 8))
    assert install_cpu_layers(model) == 2
    assert type(model[0]) is RMSNormCPU and type(model[1]) is LayerNormCPU and type(model[2]) is nn.Linear
    assert set(GroupedRMSNormCPU(64, 8).state_dict()) == {"weight"}
    assert set(SwiGLUCPU(64, 96, bias=True).state_dict()) == {"w_in.weight", "w_in.bias", "w_down.weight",
                                                              "w_down.bias"}


def test_modules_refuse_other_paths(monkeypatch):
    """With the kernels switched on there is no CPU or autograd fallback: the modules raise instead of
    computing something else. Only an explicit switch selects the upstream PyTorch forward."""
    from montlok.rdt import Mamba3HIP, RMSNormCPU, cpu_linear
    from montlok.rdt import torch_path

    x = torch.randn(2, 3, 64)
    with torch.no_grad(), pytest.raises(RuntimeError, match="must be on the ROCm device"):
        Mamba3HIP(64, d_state=16, headdim=32)(x)
    with torch.no_grad(), pytest.raises(RuntimeError, match="must be on the ROCm device"):
        RMSNormCPU(64)(x)
    with pytest.raises(RuntimeError, match="cpu_linear"):
        cpu_linear(x, torch.zeros(4, 64))
    monkeypatch.setenv("MONTLOK_CPP_LAYERS", "0")
    norm = RMSNormCPU(64)
    with torch.no_grad():
        assert torch.equal(norm(x), torch_path.rms_norm(x, norm.weight, norm.eps))
        with pytest.raises(RuntimeError, match="must be on the ROCm device"):
            Mamba3HIP(64, d_state=16, headdim=32)(x)  # the Mamba-3 kernels are still on


def test_stage2_tail_argument_checks():
    """montlok.cpp:1239-1245: the packed tail op rejects a bad depth, stream count or pack before any launch."""
    from montlok import _C

    x = torch.zeros(1, 2, 8)
    hc, mla, ffn = [x] * 8, [x] * 9, [x] * 4
    common = dict(attn_hc_eps=1e-5, attn_sinkhorn_iters=20, attn_norm_weight=x, attn_norm_eps=1e-5, kv_norm_eps=1e-5,
                  n_heads=1, head_dim=8, nope_dim=4, kv_lora_rank=8, attn_scale=1.0, ffn_hc_eps=1e-5,
                  ffn_sinkhorn_iters=20, ffn_norm_weight=x, ffn_norm_eps=1e-5)
    cases = [((0, 4, hc, mla, hc, ffn), "depth must be positive"),
             ((1, 0, hc, mla, hc, ffn), "n_streams must be positive"),
             ((1, 4, hc[:7], mla, hc, ffn), "each mHC tensor pack must contain dyn/proj/biases/alphas"),
             ((1, 4, hc, mla[:8], hc, ffn), "MLA tensor pack must contain full/tail/q/norm/kv/out/rope tensors"),
             ((1, 4, hc, mla, hc, ffn[:3]), "FFN tensor pack must contain in/out weights and biases")]
    for (depth, n, a_hc, a_mla, f_hc, a_ffn), message in cases:
        with pytest.raises(RuntimeError, match=message):
            _C.stage2_tail_forward(x, depth, n, attn_hc=a_hc, mla=a_mla, ffn_hc=f_hc, ffn=a_ffn, **common)


def test_cpu_features_keys():
    """montlok.cpp:1361-1378: the same keys as the reference's host-CPU description."""
    from montlok import _C

    info = _C.cpu_features()
    assert set(info) == {"brand", "arch", "sse2", "sse4_2", "avx", "fma", "avx2", "avx512f", "avx512dq", "avx512bw",
                         "avx512vl", "os_avx", "os_avx512"}
    assert isinstance(info["brand"], str) and info["arch"] in ("x86-64", "arm64", "other")
    assert all(isinstance(info[k], bool) for k in info if k not in ("brand", "arch"))


def _tiny_model_config(**overrides):
    model = dict(d_model=64, n_heads=2, head_dim=32, rope_head_dim=16, nope_head_dim=16, kv_lora_rank=64,
                 ffn_hidden=128, n_prelude=0, n_coda=0, core_type="two_stage", stage1_mamba_layers=1,
                 stage2_attn_layers=1, recurrent_steps=2, recurrent_drift_mode="mhc", mhc_n_streams=4,
                 mhc_sinkhorn_iters=20, mamba_d_state=16, mamba_headdim=32, mamba_expand=2, mamba_chunk_size=64,
                 use_official_mamba=True, use_morphological_rope=False, bidirectional=False, max_seq_len=64,
                 grad_ckpt_blocks=False, grad_ckpt_recurrent=True)
    model.update(overrides)
    return {"model": model, "horizons_minutes": [15, 60, 240]}


def test_model_state_dict_contract():
    """The upstream two-stage module tree (Model/two_stage.py:58-168, Model/blocks.py:120-131,
    Model/layers/mamba3_layer.py:383-445) under RDT4QuantCPU (model.py:289-305): every key and shape a
    checkpoint carries, written out from those modules."""
    from montlok.rdt import RDT4QuantCPU, RDT4QuantHIP

    assert RDT4QuantCPU is RDT4QuantHIP
    m = RDT4QuantHIP(7, _tiny_model_config())
    shapes = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    s1, s2 = "recurrent.stage1.0.", "recurrent.stage2.0."
    hc = {"pre_bias": (4,), "post_bias": (4,), "res_bias": (4, 4), "dyn_norm.weight": (64,),
          "pre_proj.weight": (4, 64), "post_proj.weight": (4, 64), "res_proj.weight": (16, 64), "pre_alpha": (),
          "post_alpha": (), "res_alpha": ()}
    expect = {"projection.weight": (64, 7), "projection.bias": (64,), "input_norm.weight": (64,),
              "input_norm.bias": (64,),
              s1 + "mamba.norm.weight": (64,), s1 + "mamba.mamba.in_proj.weight": (2 * 128 + 2 * 16 + 3 * 4 + 4, 64),
              s1 + "mamba.mamba.dt_bias": (4,), s1 + "mamba.mamba.B_bias": (4, 1, 16),
              s1 + "mamba.mamba.C_bias": (4, 1, 16), s1 + "mamba.mamba.B_norm.weight": (16,),
              s1 + "mamba.mamba.C_norm.weight": (16,), s1 + "mamba.mamba.D": (4,),
              s1 + "mamba.mamba.out_proj.weight": (64, 128), s1 + "ffn_norm.weight": (64,),
              s1 + "ffn.w_in.weight": (256, 64), s1 + "ffn.w_down.weight": (64, 128),
              s2 + "attn_norm.weight": (64,), s2 + "attn.q_proj.weight": (64, 64),
              s2 + "attn.kv_down.weight": (64, 64), s2 + "attn.kv_norm.weight": (64,),
              s2 + "attn.kv_norm.bias": (64,), s2 + "attn.kv_up.weight": (2 * 48, 64),
              s2 + "attn.k_rope_proj.weight": (16, 64), s2 + "attn.o_proj.weight": (64, 64),
              s2 + "ffn_norm.weight": (64,), s2 + "ffn.w_in.weight": (256, 64), s2 + "ffn.w_down.weight": (64, 128),
              "final_norm.weight": (64,), "head.weight": (9, 64), "head.bias": (9,)}
    for k, v in hc.items():
        expect[s2 + "attn_hc." + k] = v
        expect[s2 + "ffn_hc." + k] = v
    assert shapes == expect
    m.load_state_dict(m.state_dict(), strict=True)


def test_multi_asset_model_contract():
    """model.py:393-406: the stock inputs' projection, norm, embeddings and per-domain heads."""
    from montlok.rdt import MultiAssetRDTCPU, MultiAssetRDTHIP

    assert MultiAssetRDTCPU is MultiAssetRDTHIP
    m = MultiAssetRDTHIP(_tiny_model_config(), asset_count=5)
    shapes = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    assert shapes["projection.weight"] == (64, 57)
    assert shapes["stock_projection.weight"] == (64, 23) and shapes["stock_norm.bias"] == (64,)
    assert shapes["asset_embedding.weight"] == (5, 64) and shapes["period_embedding.weight"] == (2, 64)
    assert shapes["stock_heads.equity_daily.weight"] == (9, 64) and shapes["stock_heads.token_hour.bias"] == (9,)


def test_model_config_refusals():
    """Configurations the reference hands to upstream PyTorch are refused, never computed another way."""
    from montlok.rdt import RDT4QuantHIP

    for overrides, message in ((dict(core_type="interleaved"), "core_type"),
                               (dict(recurrent_drift_mode="none"), "recurrent_drift_mode"),
                               (dict(n_prelude=2), "prelude/coda"), (dict(use_morphological_rope=True), "morphological"),
                               (dict(use_mol=True), "mixture-of-LoRA")):
        with pytest.raises(NotImplementedError, match=message):
            RDT4QuantHIP(7, _tiny_model_config(**overrides))
    with pytest.raises(ValueError, match="use_official_mamba"):
        RDT4QuantHIP(7, _tiny_model_config(use_official_mamba=False))
    m = RDT4QuantHIP(7, _tiny_model_config())
    with pytest.raises(RuntimeError, match="ROCm device|switched off"):
        with torch.no_grad():
            m(torch.zeros(1, 4, 7), 1)


def test_switch_predicates(monkeypatch):
    """The reference's MONTLOK_CPP* switches (README.md:265-280) as this package reads them."""
    from montlok.rdt import mamba3, model

    for name in ("MONTLOK_CPP_FUSED", "MONTLOK_CPP_TAIL", "MONTLOK_CPP_NATIVE_STAGE1", "MONTLOK_CPP_NATIVE_STAGE2",
                 "MONTLOK_CPP_LAYERS"):
        monkeypatch.delenv(name, raising=False)
    monkeypatch.setenv("MONTLOK_CPP", "1")
    assert mamba3.cpp_backend() == "fused"
    assert model.tail_enabled() and model.native_stage1_enabled() and model.native_stage2_enabled()
    monkeypatch.setenv("MONTLOK_CPP_FUSED", "0")
    assert mamba3.cpp_backend() == "recurrent" and not model.native_stage1_enabled() and model.tail_enabled()
    monkeypatch.delenv("MONTLOK_CPP_FUSED")
    monkeypatch.setenv("MONTLOK_CPP_TAIL", "0")
    assert not model.tail_enabled() and model.native_stage1_enabled()
    monkeypatch.setenv("MONTLOK_CPP_NATIVE_STAGE2", "0")
    assert not model.native_stage2_enabled() and model.native_stage1_enabled()
    monkeypatch.setenv("MONTLOK_CPP_NATIVE_STAGE1", "0")
    assert not model.native_stage1_enabled()
    monkeypatch.setenv("MONTLOK_CPP", "0")
    assert mamba3.cpp_backend() is None and not model.tail_enabled()


def test_block_and_decode_stack_contract():
    """Mamba3BlockHIP carries the upstream Mamba3Layer keys (norm.weight, mamba.*); DecodeStackHIP adds the
    final norm and the head."""
    from montlok.rdt import DecodeStackHIP, Mamba3BlockHIP

    b = Mamba3BlockHIP(64, d_state=16, headdim=32, num_groups=8)
    keys = set(b.state_dict())
    assert {"norm.weight", "mamba.in_proj.weight", "mamba.out_proj.weight", "mamba.dt_bias", "mamba.D"} <= keys
    assert b.norm.num_groups == 8 and b.mamba.in_proj.weight.shape == (2 * 128 + 2 * 16 + 3 * 4 + 4, 64)
    s = DecodeStackHIP(d_model=128, n_layers=2, d_state=64, headdim=64)
    assert s.head.weight.shape == (1, 128) and len(s.layers) == 2
    with pytest.raises(ValueError, match="expects"):
        b(torch.zeros(2, 3, 32))


def test_mla_pack_cache_holds_weights_weakly(monkeypatch):
    """The packed-weight cache keys on (object, data_ptr, _version) and holds its weights only weakly:
    a `.data` swap misses the cache, and deleting the weights drops their entry (CPU tensors and a stub
    packer stand in for the device)."""
    import gc

    from montlok import _C

    made = []

    def fake_pack(a, b, c, *rest):
        made.append((a.data_ptr(), b.data_ptr(), c.data_ptr()))
        return torch.zeros(1)

    class _Stream:
        def __eq__(self, other):
            return True

    monkeypatch.setattr(_C, "mla_pack_weights", fake_pack)
    monkeypatch.setattr(_C.torch.cuda, "current_stream", lambda device=None: _Stream())
    monkeypatch.setattr(_C.torch.cuda, "is_current_stream_capturing", lambda: False)
    monkeypatch.setattr(_C, "_MLA_PACKS", [])
    ws = [torch.zeros(4), torch.zeros(5), torch.zeros(6)]
    first = _C._mla_packed(*ws, 8, 32, 16, 64)
    assert _C._mla_packed(*ws, 8, 32, 16, 64) is first and len(made) == 1
    ws[1].add_(1.0)  # in-place through the tensor: _version moves
    assert _C._mla_packed(*ws, 8, 32, 16, 64) is not first and len(made) == 2
    ws[2].data = torch.ones(6)  # data swap: same object and _version, new data_ptr
    _C._mla_packed(*ws, 8, 32, 16, 64)
    assert len(made) == 3
    assert len(_C._MLA_PACKS) == 3
    del ws
    gc.collect()
    _C._mla_packed(torch.zeros(4), torch.zeros(5), torch.zeros(6), 8, 32, 16, 64)
    assert len(_C._MLA_PACKS) == 1, "entries of deleted weights must be dropped"

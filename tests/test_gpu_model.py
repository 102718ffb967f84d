"""GPU parity of the model-level drop-in (python/montlok/rdt/model.py:289-417):
RDT4QuantHIP's forward (native stage 1, native stage-2 tail, quantile head)
against the same chain of oracle ops, 1e-5 normwise; the tail path against
the last row of the full recurrence; and the multi-asset stock path."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close
from test_gpu_modules import _mamba_oracle, _np
from test_gpu_stage2 import _oracle_tail
from test_modules import _tiny_model_config

pytestmark = pytest.mark.gpu


def _model(cls=None, seed=0, **overrides):
    from montlok.rdt import RDT4QuantHIP

    torch.manual_seed(seed)
    cfg = _tiny_model_config(d_model=128, n_heads=4, ffn_hidden=192, stage1_mamba_layers=2, **overrides)
    m = (cls or RDT4QuantHIP)(*((7, cfg) if cls is None else (cfg, 3))).eval()
    with torch.no_grad():
        for name, p in m.named_parameters():
            if name.endswith(("norm.weight", "norm.bias")) or "_norm." in name:
                p.add_(0.1 * torch.randn_like(p))
            elif name.endswith(("pre_alpha", "post_alpha", "res_alpha")):
                p.fill_(0.7)
            elif name.endswith("res_bias"):
                p.normal_()
            elif name.endswith(("pre_proj.weight", "post_proj.weight", "res_proj.weight")):
                p.normal_(0.0, 128 ** -0.5)
            elif name.endswith("bias") and p.dim() == 1 and "mamba" not in name:
                p.normal_(0.0, 0.1)
    return m


def _oracle_stage1(oracle, core, x):
    hidden = x
    layers = list(core.stage1)
    first = layers[0].mamba.norm
    mamba_in = oracle.rms_norm(hidden, _np(first.weight), first.eps, first.num_groups)
    for i, layer in enumerate(layers):
        m = _mamba_oracle(oracle, layer.mamba.mamba, mamba_in)
        hidden, normed = oracle.add_rms_norm(hidden, m, _np(layer.ffn_norm.weight), layer.ffn_norm.eps, 1)
        f = layer.ffn
        ffn = oracle.linear(oracle.swiglu(oracle.linear(normed, _np(f.w_in.weight))), _np(f.w_down.weight))
        if i + 1 == len(layers):
            hidden = hidden + ffn
        else:
            nxt = layers[i + 1].mamba.norm
            hidden, mamba_in = oracle.add_rms_norm(hidden, ffn, _np(nxt.weight), nxt.eps, nxt.num_groups)
    return hidden


def _oracle_head(oracle, m, hidden, head, rows):
    last = oracle.rms_norm(np.ascontiguousarray(hidden[:, -1]), _np(m.final_norm.weight), m.final_norm.eps, 1)
    raw = torch.from_numpy(oracle.linear(last, _np(head.weight), _np(head.bias))).reshape(-1, rows, 3)
    return m._quantiles(raw).numpy()


@pytest.mark.parametrize("depth,L", [(1, 24), (3, 40)])
def test_model_forward_vs_oracle(dev, oracle, depth, L):
    m = _model(seed=depth)
    x = torch.randn(3, L, 7, generator=torch.Generator().manual_seed(depth))
    with torch.no_grad():
        got, rms = m.to(dev)(x.to(dev), depth)
    m = m.cpu()
    embedded = oracle.layer_norm(oracle.linear(x.numpy(), _np(m.projection.weight), _np(m.projection.bias)),
                                 _np(m.input_norm.weight), _np(m.input_norm.bias), m.input_norm.eps)
    backbone = _oracle_stage1(oracle, m.recurrent, embedded)
    hidden = _oracle_tail(oracle, m.recurrent.stage2[0], backbone, depth)
    assert_close(got, _oracle_head(oracle, m, hidden, m.head, 3), tol=1e-5, name=f"quantiles depth {depth}")
    assert abs(rms.item() - float(np.sqrt(np.mean(hidden.astype(np.float64) ** 2)))) <= 1e-5 * (1 + rms.item())
    q = got.cpu()
    assert bool((q[..., 0] <= q[..., 1]).all() and (q[..., 1] <= q[..., 2]).all())


def test_model_tail_equals_full_recurrence(dev):
    """model.py:1-8: the tail path is row for row the arithmetic of the full pass."""
    m = _model(seed=5).to(dev)
    x = torch.randn(2, 32, 7, generator=torch.Generator().manual_seed(7)).to(dev)
    with torch.no_grad():
        full, info = m.encode(x, 2)
        tail = m._hidden_tail(m._embed(x), 2)
    assert info["steps_used"] == 2
    assert_close(tail[:, 0], full[:, -1], tol=1e-6, name="tail vs full recurrence")


def test_model_parameter_packs_follow_load_state_dict(dev):
    """model.py:310-323: packs are rebuilt after load_state_dict, so new weights take effect."""
    m = _model(seed=2).to(dev)
    other = _model(seed=3).to(dev)
    x = torch.randn(2, 16, 7, generator=torch.Generator().manual_seed(1)).to(dev)
    with torch.no_grad():
        a = m(x, 1)[0]
        m.load_state_dict(other.state_dict())
        b = m(x, 1)[0]
        c = other(x, 1)[0]
    assert torch.equal(b, c) and not torch.equal(a, b)


def test_multi_asset_stock_path(dev, oracle):
    from montlok.rdt import MultiAssetRDTHIP

    m = _model(MultiAssetRDTHIP, seed=4)
    x = torch.randn(2, 24, 23, generator=torch.Generator().manual_seed(2))
    asset = torch.tensor([0, 2])
    with torch.no_grad():
        got, _ = m.to(dev)(x.to(dev), 2, domain="equity_daily", asset_id=asset.to(dev))
        crypto, _ = m(torch.randn(2, 24, 57, device=dev), 1)
    assert tuple(got.shape) == (2, 3, 3) and tuple(crypto.shape) == (2, 3, 3)
    m = m.cpu()
    projected = oracle.linear(x.numpy(), _np(m.stock_projection.weight), _np(m.stock_projection.bias))
    projected = projected + _np(m.asset_embedding.weight)[asset.numpy()][:, None] + _np(m.period_embedding.weight)[0]
    embedded = oracle.layer_norm(projected.astype(np.float32), _np(m.stock_norm.weight), _np(m.stock_norm.bias),
                                 m.stock_norm.eps)
    hidden = _oracle_tail(oracle, m.recurrent.stage2[0], _oracle_stage1(oracle, m.recurrent, embedded), 2)
    expect = _oracle_head(oracle, m, hidden, m.stock_heads["equity_daily"], 3)
    assert_close(got, expect, tol=1e-5, name="stock quantiles")
    with pytest.raises(ValueError, match="typed stock domain"):
        with torch.no_grad():
            m.to(dev)(x.to(dev), 1, domain="bonds", asset_id=asset.to(dev))

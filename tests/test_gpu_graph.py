"""The mHC step captured in a HIP graph: several replays, with eager work and
synchronisations in between, each equal to the eager result bit for bit."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_mhc_step_graph_replays_match_eager(dev):
    from montlok import _C

    g = torch.Generator(device="cpu").manual_seed(3)
    n, d, B, L = 4, 128, 8, 64
    s = torch.randn(B, L, n, d, generator=g).to(dev)
    p = ((torch.rand(d, generator=g) + 0.5).to(dev), 1e-5,
         (torch.randn(2 * n + n * n, d, generator=g, dtype=torch.float64) / d ** 0.5).to(dev),
         torch.randn(n, generator=g).to(dev), torch.randn(n, generator=g).to(dev), torch.randn(n, n, generator=g).to(dev),
         torch.tensor(0.7, device=dev), torch.tensor(0.6, device=dev), torch.tensor(0.8, device=dev), 20)
    agg, pre, post, res = _C.mhc_prepare(s, *p)
    new = _C.mhc_combine(s, res, post, agg)
    torch.cuda.synchronize()
    expect = [t.clone() for t in (agg, pre, post, res, new)]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out = list(_C.mhc_prepare(s, *p))
        out.append(_C.mhc_combine(s, out[3], out[2], out[0]))
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = list(_C.mhc_prepare(s, *p))
        out.append(_C.mhc_combine(s, out[3], out[2], out[0]))
    for replay in range(4):
        for t in out:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(out, expect):
            assert torch.equal(a, b), f"replay {replay}"
        _ = (s * 2).sum().item()  # unrelated eager work between replays

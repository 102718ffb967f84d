"""The allocation-free recurrence entry point (mlk_mamba3_siso_recurrent_noalloc,
no counterpart in the reference) against mlk_mamba3_siso_recurrent, which takes
a caller workspace: bit for bit, on two calls in a row (the second smaller, so
it runs over what the first left in the static scratch), with strided views,
a size beyond the static scratch rejected before any launch, calls on two
streams ordered by the library, and the call captured in a HIP graph."""

from __future__ import annotations

import pytest
import torch

from helpers import assert_bitwise

pytestmark = pytest.mark.gpu


def _inputs(g, B, L, H, N, D, dev):
    q = torch.randn(B, L, H, N, generator=g).to(dev)
    k = torch.randn(B, L, H, N, generator=g).to(dev)
    # v and the gate as strided views of wider rows, as mamba3_siso_forward passes them.
    wide = torch.randn(B, L, H, 2 * D, generator=g).to(dev)
    v, z = wide[..., :D], wide[..., D:]
    gate = z * torch.sigmoid(z)
    dt = torch.nn.functional.softplus(torch.randn(B, L, H, generator=g) - 3).to(dev)
    adt = -torch.rand(B, L, H, generator=g).to(dev) * dt
    trap = torch.randn(B, L, H, generator=g).to(dev)
    skip = torch.randn(H, generator=g).to(dev)
    return q, k, v, gate, adt, dt, trap, skip


def test_noalloc_equals_workspace_entry_point(dev):
    from montlok import _C

    g = torch.Generator().manual_seed(31)
    shapes = [(64, 32, 4, 16, 32), (3, 45, 2, 64, 64)]  # the second call is smaller than the first
    for B, L, H, N, D in shapes:
        args = _inputs(g, B, L, H, N, D, dev)
        expect = _C.mamba3_siso_recurrent(*args)
        got = _C.mamba3_siso_recurrent_noalloc(*args)
        torch.cuda.synchronize()
        assert got.shape == (B, L, H, D)
        assert torch.isfinite(got).all().item()
        assert_bitwise(got, expect.cpu().numpy(), f"noalloc vs workspace recurrence {B}x{L}x{H}")


def test_noalloc_rejects_sizes_beyond_its_scratch(dev):
    from montlok import _C

    B, L, H = 1, 699_051, 1  # B * L * H one past the static scratch's capacity
    q = torch.zeros(B, L, H, 16, device=dev)
    v = torch.zeros(B, L, H, 16, device=dev)
    c = torch.zeros(B, L, H, device=dev)
    with pytest.raises(RuntimeError, match="exceeds the static scratch"):
        _C.mamba3_siso_recurrent_noalloc(q, q, v, v, c, c, c, torch.zeros(H, device=dev))


def test_noalloc_calls_on_two_streams_are_ordered(dev):
    """A long call on one stream, then at once a shorter one on another: the second call's coefficients
    would overwrite the first's while the first still reads them, unless the library orders the two."""
    from montlok import _C

    g = torch.Generator().manual_seed(41)
    big = _inputs(g, 16, 2048, 16, 16, 32, dev)  # B * L * H = 524,288 of the scratch's 699,050
    small = _inputs(g, 8, 512, 4, 16, 32, dev)
    expect_big = _C.mamba3_siso_recurrent(*big)
    expect_small = _C.mamba3_siso_recurrent(*small)
    torch.cuda.synchronize()
    for trial in range(3):
        sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
        sa.wait_stream(torch.cuda.current_stream())
        sb.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(sa):
            got_big = _C.mamba3_siso_recurrent_noalloc(*big)
        with torch.cuda.stream(sb):
            got_small = _C.mamba3_siso_recurrent_noalloc(*small)
        torch.cuda.synchronize()
        assert_bitwise(got_big, expect_big.cpu().numpy(), f"first call, stream A, trial {trial}")
        assert_bitwise(got_small, expect_small.cpu().numpy(), f"second call, stream B, trial {trial}")


def test_noalloc_under_graph_capture(dev):
    """One eager call (the per-device set-up), then the call captured in a graph: every replay, with other
    eager noalloc calls between them that overwrite the scratch, equals the workspace form bit for bit."""
    from montlok import _C

    g = torch.Generator().manual_seed(43)
    args = _inputs(g, 8, 96, 4, 16, 32, dev)
    other = _inputs(g, 4, 200, 2, 32, 64, dev)
    expect = _C.mamba3_siso_recurrent(*args).cpu().numpy()
    expect_other = _C.mamba3_siso_recurrent(*other).cpu().numpy()
    _C.mamba3_siso_recurrent_noalloc(*args)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _C.mamba3_siso_recurrent_noalloc(*args)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = _C.mamba3_siso_recurrent_noalloc(*args)
    for replay in range(4):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert_bitwise(out, expect, f"graph replay {replay}")
        eager = _C.mamba3_siso_recurrent_noalloc(*other)
        torch.cuda.synchronize()
        assert_bitwise(eager, expect_other, f"eager call after replay {replay}")

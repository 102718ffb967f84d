"""The allocation-free recurrence entry point (mlk_mamba3_siso_recurrent_noalloc,
no counterpart in the reference) against mlk_mamba3_siso_recurrent, which takes
a caller workspace: bit for bit, on two calls in a row (the second smaller, so
it runs over what the first left in the static scratch), with strided views,
and a size beyond the static scratch rejected before any launch."""

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

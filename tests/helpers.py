"""Comparison helpers shared by the tests.

Tolerance definition used everywhere: the normwise relative error
max|actual - expected| / max|expected| must not exceed `tol` (1e-5 for fp32
paths, 2e-2 for bf16-weight paths). The reference's own form,
max|diff| <= tol * (1 + max|expected|) (tests/rdt/test_rdt_kernels.py:127),
is reported alongside. Integer/index outputs are compared with ==.
"""

from __future__ import annotations

import numpy as np

FP32_TOL = 1e-5
BF16_TOL = 2e-2


def to_np(a):
    try:
        import torch

        if isinstance(a, torch.Tensor):
            return a.detach().float().cpu().numpy() if a.dtype != torch.float64 else a.detach().cpu().numpy()
    except ImportError:  # pragma: no cover
        pass
    return np.asarray(a)


def rel_err(actual, expected) -> float:
    a = to_np(actual).astype(np.float64)
    e = to_np(expected).astype(np.float64)
    assert a.shape == e.shape, f"shape {a.shape} != {e.shape}"
    if e.size == 0:
        return 0.0
    scale = np.abs(e).max()
    diff = np.abs(a - e).max()
    return float(diff / scale) if scale > 0 else float(diff)


def assert_close(actual, expected, tol=FP32_TOL, name=""):
    a = to_np(actual)
    assert np.isfinite(a).all(), f"{name}: non-finite values"
    err = rel_err(actual, expected)
    assert err <= tol, f"{name}: normwise relative error {err:.3e} > {tol:.1e}"
    return err


def bit_mismatches(actual, expected) -> int:
    a = np.ascontiguousarray(to_np(actual), dtype=np.float32)
    e = np.ascontiguousarray(to_np(expected), dtype=np.float32)
    assert a.shape == e.shape
    return int((a.view(np.uint32) != e.view(np.uint32)).sum())


def assert_bitwise(actual, expected, name=""):
    n = bit_mismatches(actual, expected)
    assert n == 0, f"{name}: {n} of {to_np(expected).size} elements differ bitwise"

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
# bf16 kernels against the float64 restatement of their roundings (tests/bf16_emu.py): the median
# output row agrees to fp32 precision (EMU_ROW_MEDIAN_TOL; measured at most 1.2e-7, while against
# the fp32 oracle the median row is off by ~3e-4); the normwise bound (EMU_TOL) leaves room for
# the rare operand that the matrix cores' fp32 accumulation order or the hardware exp2 moves
# across a bf16 rounding boundary (one bf16 ulp of one operand, largest in the first rows of a
# causal window where a key carries much of the softmax weight; measured at most 4.4e-4).
EMU_TOL = 1e-3
EMU_ROW_MEDIAN_TOL = 1e-6


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


def row_errors(actual, expected):
    """Per-row normwise errors max_j |a_ij - e_ij| / max|e| over the last dimension, as a flat array."""
    a = to_np(actual).astype(np.float64)
    e = to_np(expected).astype(np.float64)
    assert a.shape == e.shape
    scale = np.abs(e).max()
    return (np.abs(a - e).reshape(-1, a.shape[-1]).max(-1) / (scale if scale > 0 else 1.0))


def assert_emulated(actual, expected, name="", tol=None, row_median_tol=None):
    """A bf16 kernel's output against the float64 restatement of its roundings: normwise <= EMU_TOL and
    the median row's normwise error <= EMU_ROW_MEDIAN_TOL. Returns (normwise, median row error)."""
    tol = EMU_TOL if tol is None else tol
    row_median_tol = EMU_ROW_MEDIAN_TOL if row_median_tol is None else row_median_tol
    a = to_np(actual)
    assert np.isfinite(a).all(), f"{name}: non-finite values"
    err = rel_err(actual, expected)
    med = float(np.median(row_errors(actual, expected)))
    assert err <= tol, f"{name}: normwise relative error {err:.3e} > {tol:.1e}"
    assert med <= row_median_tol, f"{name}: median row error {med:.3e} > {row_median_tol:.1e}"
    return err, med

"""Comparison criteria shared by the CPU and GPU tests.

fp32 storage: per row, max|got - ref| / max|ref| <= 1e-5 (y, dx).
bf16 storage: the same form at 1e-2.
dgamma: max_j |got_j - ref_j| / max_j |ref_j| <= the same tolerance.  An
element-wise relative bound on dgamma is not meaningful: each dgamma_j is a
sum of R terms of random sign, and the columns whose sum happens to land near
zero carry a relative rounding error no fp32 accumulation can meet.
"""
from __future__ import annotations

import numpy as np

TOL_F32 = 1e-5
TOL_BF16 = 1e-2


def row_rel_err(got, ref) -> float:
    """max over rows of max|got-ref| / max|ref| (absolute error for all-zero rows)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if ref.size == 0:
        return 0.0
    cols = ref.shape[-1]
    g = got.reshape(-1, cols)
    r = ref.reshape(-1, cols)
    num = np.max(np.abs(g - r), axis=1)
    den = np.max(np.abs(r), axis=1)
    err = np.where(den > 0, num / np.where(den > 0, den, 1.0), num)
    if np.any(~np.isfinite(g)) and not np.array_equal(np.isnan(g), np.isnan(r)):
        return float("inf")
    return float(np.max(err))


def vec_rel_err(got, ref) -> float:
    got = np.asarray(got, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    if ref.size == 0:
        return 0.0
    den = np.max(np.abs(ref))
    num = np.max(np.abs(got - ref))
    if not np.all(np.isfinite(got)):
        return float("inf")
    return float(num / den) if den > 0 else float(num)

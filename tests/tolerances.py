"""Comparison criteria shared by the CPU and GPU tests.

fp32 storage: per row, max|got - ref| / max|ref| <= 1e-5 (y, dx).
bf16 storage: the same form at 1e-2.
dx: per row, max|got - ref| / (max_j r|g_j| + max_j r^3 |x_j dot| / D), i.e.
relative to the two terms whose difference dx is (g = dy*gamma, dot = sum g x).
For ordinary rows this is within a small factor of max|dx|; for rows where
they cancel (a width-1 row, where dx = g eps r^3, or dy*gamma parallel to x)
it is the only bound an fp32 computation can meet.
dgamma: max_j |got_j - ref_j| / max_j |ref_j| <= the same tolerance, and
element-wise against each column's own condition: |got_j - ref_j| <=
tol * sum_i |dy_ij x_ij r_i| (dgamma_elem_err).  A plain element-wise relative
bound |got_j - ref_j| / |ref_j| is not meaningful: each dgamma_j is a sum of R
terms of random sign, and the columns whose sum happens to land near zero
carry a relative rounding error no fp32 accumulation can meet; measured
against the sum of its terms' magnitudes, every column is held to the bar.
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


def dx_scale(x, gamma, dy, eps):
    """Per-row magnitude of the terms of dx = r*g - x*r^3*dot/D (fp64)."""
    x = np.asarray(x, dtype=np.float64)
    cols = x.shape[-1]
    x = x.reshape(-1, cols)
    g = np.asarray(dy, dtype=np.float64).reshape(-1, cols)
    if gamma is not None:
        g = g * np.asarray(gamma, dtype=np.float64).reshape(1, cols)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=1) + eps)
    dot = np.sum(g * x, axis=1)
    t1 = r * np.max(np.abs(g), axis=1)
    t2 = r ** 3 * np.max(np.abs(x), axis=1) * np.abs(dot) / cols
    return t1 + t2


def dx_rel_err(got, ref, x, gamma, dy, eps) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if ref.size == 0:
        return 0.0
    cols = ref.shape[-1]
    num = np.max(np.abs(got.reshape(-1, cols) - ref.reshape(-1, cols)), axis=1)
    if not np.all(np.isfinite(got)):
        return float("inf")
    den = dx_scale(x, gamma, dy, eps)
    return float(np.max(np.where(den > 0, num / np.where(den > 0, den, 1.0), num)))


def dgamma_elem_err(got, ref, x, dy, inv_rms) -> float:
    """max_j |got_j - ref_j| / sum_i |dy_ij x_ij r_i| (fp64): each dgamma column
    against the magnitude of the terms it sums (absolute where they are all 0)."""
    got = np.asarray(got, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    if ref.size == 0:
        return 0.0
    if not np.all(np.isfinite(got)):
        return float("inf")
    cols = ref.size
    x = np.asarray(x, dtype=np.float64).reshape(-1, cols)
    dy = np.asarray(dy, dtype=np.float64).reshape(-1, cols)
    r = np.asarray(inv_rms, dtype=np.float64).reshape(-1, 1)
    den = np.sum(np.abs(dy * x * r), axis=0)
    num = np.abs(got - ref)
    return float(np.max(np.where(den > 0, num / np.where(den > 0, den, 1.0), num)))

"""CPU oracle for the RMSNorm layer path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this package, and only as the checker (or the timed CPU baseline).  The
product (cgadimpl_amd) never imports it.

Functions here bind ``liboracle_rmsnorm.so`` built from ``rmsnorm_oracle.c``,
a restatement of the reference's op sequence (see that file's header for the
file:line citations).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

from . import build as _build

HERE = os.path.dirname(os.path.abspath(__file__))

_libs: dict = {}


def load(mutation: int = 0, rebuild: bool = False) -> ctypes.CDLL:
    """Load (building if needed) the oracle; mutation > 0 plants a mistake."""
    if mutation in _libs and not rebuild:
        return _libs[mutation]
    path = _build.lib_path(mutation)
    if rebuild or not os.path.exists(path) or (
            os.path.getmtime(path) < os.path.getmtime(_build.SRC)):
        _build.build(mutation)
    h = ctypes.CDLL(path)
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    h.oracle_rmsnorm_fwd_f32.restype = ctypes.c_int
    h.oracle_rmsnorm_fwd_f32.argtypes = [P, P, P, P, P, I64, I64, ctypes.c_float]
    h.oracle_rmsnorm_bwd_f32.restype = ctypes.c_int
    h.oracle_rmsnorm_bwd_f32.argtypes = [P, P, P, P, P, P, I64, I64, ctypes.c_int]
    h.oracle_rmsnorm_fwd_bf16.restype = ctypes.c_int
    h.oracle_rmsnorm_fwd_bf16.argtypes = [P, P, P, P, I64, I64, ctypes.c_float]
    h.oracle_rmsnorm_bwd_bf16.restype = ctypes.c_int
    h.oracle_rmsnorm_bwd_bf16.argtypes = [P, P, P, P, P, P, I64, I64, ctypes.c_int]
    h.oracle_rmsnorm_truth_f64.restype = None
    h.oracle_rmsnorm_truth_f64.argtypes = [P, P, P, P, P, P, P, I64, I64, ctypes.c_double]
    h.oracle_bf16_encode.argtypes = [P, P, I64]
    h.oracle_bf16_decode.argtypes = [P, P, I64]
    h.oracle_set_threads.argtypes = [ctypes.c_int]
    h.oracle_mutation.restype = ctypes.c_int
    _libs[mutation] = h
    return h


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


def set_threads(n: int, mutation: int = 0) -> None:
    load(mutation).oracle_set_threads(int(n))


def fwd(x, gamma, eps: float, mutation: int = 0, want_xhat: bool = False):
    """Reference-order forward.  float32 arrays, or uint16 bf16 bit patterns.

    Returns (y, inv_rms) or (y, inv_rms, xhat) for fp32 with want_xhat.
    """
    h = load(mutation)
    cols = x.shape[-1]
    rows = x.size // cols if cols else 0
    inv = np.empty(x.shape[:-1], dtype=np.float32)
    if x.dtype == np.uint16:
        xc, gc = _c(x, np.uint16), _c(gamma, np.uint16)
        y = np.empty_like(xc)
        rc = h.oracle_rmsnorm_fwd_bf16(_p(xc), _p(gc), _p(y), _p(inv), rows, cols, eps)
        assert rc == 0, rc
        return y, inv
    xc, gc = _c(x, np.float32), _c(gamma, np.float32)
    y = np.empty_like(xc)
    xhat = np.empty_like(xc) if want_xhat else None
    rc = h.oracle_rmsnorm_fwd_f32(_p(xc), _p(gc), _p(y), _p(inv), _p(xhat), rows, cols, eps)
    assert rc == 0, rc
    return (y, inv, xhat) if want_xhat else (y, inv)


def bwd(x, gamma, inv_rms, dy, mutation: int = 0, dx=None, dgamma=None,
        accumulate: bool = False, want_dgamma: bool = True):
    """Reference-order backward; returns (dx, dgamma).  dgamma is float32."""
    h = load(mutation)
    cols = x.shape[-1]
    rows = x.size // cols if cols else 0
    inv = _c(inv_rms, np.float32)
    if want_dgamma:
        dgamma = np.zeros(cols, dtype=np.float32) if dgamma is None else \
            np.ascontiguousarray(dgamma, dtype=np.float32).copy()
    else:
        dgamma = None
    if x.dtype == np.uint16:
        xc, gc, dyc = _c(x, np.uint16), _c(gamma, np.uint16), _c(dy, np.uint16)
        dxo = np.zeros_like(xc) if dx is None else np.ascontiguousarray(dx, np.uint16).copy()
        rc = h.oracle_rmsnorm_bwd_bf16(_p(xc), _p(gc), _p(inv), _p(dyc), _p(dxo), _p(dgamma),
                                       rows, cols, int(accumulate))
    else:
        xc, gc, dyc = _c(x, np.float32), _c(gamma, np.float32), _c(dy, np.float32)
        dxo = np.zeros_like(xc) if dx is None else np.ascontiguousarray(dx, np.float32).copy()
        rc = h.oracle_rmsnorm_bwd_f32(_p(xc), _p(gc), _p(inv), _p(dyc), _p(dxo), _p(dgamma),
                                      rows, cols, int(accumulate))
    assert rc == 0, rc
    return dxo, dgamma


def truth(x, gamma, dy, eps: float, mutation: int = 0):
    """fp64 closed form: returns (y, inv_rms, dx, dgamma) as float64 arrays."""
    h = load(mutation)
    x64 = np.ascontiguousarray(x, dtype=np.float64)
    g64 = None if gamma is None else np.ascontiguousarray(gamma, dtype=np.float64)
    dy64 = None if dy is None else np.ascontiguousarray(dy, dtype=np.float64)
    cols = x64.shape[-1]
    rows = x64.size // cols if cols else 0
    y = np.empty_like(x64)
    inv = np.empty(x64.shape[:-1], dtype=np.float64)
    dx = np.empty_like(x64) if dy is not None else None
    dg = np.empty(cols, dtype=np.float64) if dy is not None else None
    h.oracle_rmsnorm_truth_f64(_p(x64), _p(g64), _p(dy64), _p(y), _p(inv), _p(dx), _p(dg),
                               rows, cols, eps)
    return y, inv, dx, dg


def bf16_encode(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    load().oracle_bf16_encode(_p(a), _p(out), a.size)
    return out


def bf16_decode(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    load().oracle_bf16_decode(_p(bits), _p(out), bits.size)
    return out


# ---- RMSNorm + linear layer (configuration c5) --------------------------------
# The reference composes the layer from graph ops: h = rms(x) * gamma
# (normalization.cpp:23-35, arithmetic.cpp:31-39), y = matmul(h, W)
# (cgadimpl/src/ops/linalg.cpp:12-20), and its VJP runs vjp_MatMul
# (cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:258-263: dA += gy B^T,
# dB += A^T gy) before the RMSNorm rules.  Restated here with bf16 storage of
# x, gamma, W, h, y, dy and dh (values rounded to nearest even where the graph
# stores them), products in float64, dW returned in float32.

def matmul_f64(a, b):
    """A @ B in float64 (the textbook product; numpy's routine)."""
    return np.asarray(a, np.float64) @ np.asarray(b, np.float64)


def linear_fwd(h_bits, w_bits):
    """y = h W for bf16 bit patterns; returns y as bf16 bits."""
    return bf16_encode(matmul_f64(bf16_decode(h_bits), bf16_decode(w_bits)).astype(np.float32))


def linear_bwd(h_bits, w_bits, dy_bits):
    """vjp_MatMul: dh = dy W^T (bf16 bits), dW = h^T dy (float32)."""
    h, w, dy = bf16_decode(h_bits), bf16_decode(w_bits), bf16_decode(dy_bits)
    dh = bf16_encode(matmul_f64(dy, w.T).astype(np.float32))
    dw = matmul_f64(h.T, dy).astype(np.float32)
    return dh, dw


def rmsnorm_linear_layer(x_bits, gamma_bits, w_bits, dy_bits, eps):
    """Forward + VJP of matmul(rms_norm(x) * gamma, W) seeded with dy.

    Returns dict(h, inv_rms, y, dh, dx, dgamma, dW): bf16 bits for h, y, dh,
    dx; float32 for inv_rms, dgamma, dW.
    """
    h, inv = fwd(x_bits, gamma_bits, eps)
    y = linear_fwd(h, w_bits)
    dh, dw = linear_bwd(h, w_bits, dy_bits)
    dx, dg = bwd(x_bits, gamma_bits, inv, dh)
    return {"h": h, "inv_rms": inv, "y": y, "dh": dh, "dx": dx, "dgamma": dg, "dW": dw}

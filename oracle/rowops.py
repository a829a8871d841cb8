"""CPU restatement of cgadimpl's row ops beside RMSNorm -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker.  The product (cgadimpl_amd) never
imports it and has no CPU fallback built on it.

Restated, expression by expression in the reference's order (paths relative
to the reference tree):

  laynor_nodeops          cgadimpl/src/ops/normalization.cpp:10-22
      mean = reduce_mean(x, {-1}, keepdim); xm = x - mean;
      var = reduce_mean(xm * xm); y = xm / sqrt(var + 1e-5f); tape {var, mean}
  vjp_LayerNorm           cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:351-365
  softmax_row_nodeops     cgadimpl/src/ops/reduction.cpp:42-53
      m = reduce_max(z); e = exp(z - m); s = reduce_sum(e); y = e / s
  vjp_SoftmaxRow          autodiff_vjp_ops.cpp:421-428   dz += y * (gy - sum(y * gy))
  logsumexp_row_nodeops   reduction.cpp:54-66            y = log(sum(exp(z - m))) + m
  vjp_LogSumExpRow        autodiff_vjp_ops.cpp:430-440   dz += gy * softmax(z) (recomputed)
  jvp_SoftmaxRow          cgadimpl/src/autodiff/autodiff_jvp_ops.cpp:411-420
  jvp_LogSumExpRow        autodiff_jvp_ops.cpp:421-434   ty = sum(softmax(z) * tz)
  jvp_RMSNorm             autodiff_jvp_ops.cpp:366-379, corrected:
      the reference returns T/rms - y*dot/(rms*N) with rms = tape[0], which
      rms_nodeops fills with 1/sqrt(mean(x^2)+eps) (normalization.cpp:26-29);
      the derivative of y = x*r is T*r - y*r*dot/N with dot = sum(T*y)
  jvp_Mul                 autodiff_jvp_ops.cpp:24-31     (tA * B) + (A * tB), for gamma
  mul_nodeops             cgadimpl/src/ops/arithmetic.cpp:31-39  y = a * b (broadcasting)
  vjp_Mul                 autodiff_vjp_ops.cpp:54-59     dA += reduce_for_broadcast(gy * B, A)
  reduce_for_broadcast    autodiff_vjp_ops.cpp:15-35     sum over the grad axes whose aligned
      target axis is missing, or is 1 where the grad's is not (keepdim), then reshape

Arithmetic is done in `dt` (float32 for the parity tests, float64 for the
pinning checks); each op materialises its result as the reference graph does.
As in the C oracle (rmsnorm_oracle.c), reductions accumulate in float64 and
round to `dt` once, because OwnTensor's accumulation order is not in the
checkout.  bf16 storage: inputs are widened to float32, the float32 path
runs, and outputs are rounded to bf16 (round to nearest even).

`mut` plants one known mistake (tests only; 0 = none):
  1  LayerNorm variance divides by D-1         2  LayerNorm eps dropped
  3  LayerNorm VJP: d_mean sign flipped        4  LayerNorm VJP: 2/D term dropped
  5  softmax divides by max(e), not sum(e)     6  softmax VJP: y*gy - dot
  7  log-sum-exp drops the + max               8  log-sum-exp VJP: no / sum
  9  RMSNorm JVP as the reference wrote it (T / r instead of T * r)
 10  RMSNorm JVP: gamma tangent term dropped
 11  reduce_for_broadcast sums only the missing leading axes, not the extent-1 ones
 12  reduce_for_broadcast aligns the shapes at the leading axis instead of the trailing one
"""
from __future__ import annotations

import numpy as np

from . import bf16_decode, bf16_encode


def _rsum(a):
    """reduce_sum(a, {-1}, keepdim) accumulated in float64, rounded once."""
    return np.sum(a, axis=-1, keepdims=True, dtype=np.float64).astype(a.dtype)


def _rmean(a, div=None):
    d = a.shape[-1] if div is None else div
    return (np.sum(a, axis=-1, keepdims=True, dtype=np.float64) / d).astype(a.dtype)


def _rmax(a):
    return np.max(a, axis=-1, keepdims=True)


# ---- LayerNorm -------------------------------------------------------------------

def layernorm_fwd(x, eps=1e-5, dt=np.float32, mut=0):
    """normalization.cpp:10-22.  Returns (y, mean, var), mean/var keepdim."""
    x = np.asarray(x, dt)
    D = x.shape[-1]
    mean = _rmean(x)
    xm = x - mean
    var = _rmean(xm * xm, D - 1 if mut == 1 else None)
    e = dt(0.0) if mut == 2 else dt(eps)
    y = xm / np.sqrt(var + e)
    return y, mean, var


def layernorm_bwd(x, mean, var, gy, eps=1e-5, dt=np.float32, mut=0):
    """autodiff_vjp_ops.cpp:351-365 (eps: the forward's, 1e-5 in the reference)."""
    x, mean, var, gy = (np.asarray(a, dt) for a in (x, mean, var, gy))
    D = x.shape[-1]
    std_inv = dt(1.0) / np.sqrt(var + dt(eps))
    d_xhat = gy * std_inv
    d_var = _rsum(gy * (x - mean) * dt(-0.5) * (std_inv * std_inv * std_inv))
    d_mean = _rsum(gy * (std_inv * dt(-1.0))) + d_var * _rsum((x - mean) * dt(-2.0)) / dt(D)
    if mut == 3:
        d_mean = -d_mean
    term = d_var * (x - mean) * (dt(2.0) / dt(D))
    if mut == 4:
        term = np.zeros_like(term)
    return d_xhat + term + d_mean / dt(D)


# ---- softmax / log-sum-exp ----------------------------------------------------------

def softmax_fwd(z, dt=np.float32, mut=0):
    """reduction.cpp:42-53."""
    z = np.asarray(z, dt)
    m = _rmax(z)
    e = np.exp(z - m)
    s = _rmax(e) if mut == 5 else _rsum(e)
    return e / s


def softmax_bwd(y, gy, dt=np.float32, mut=0):
    """autodiff_vjp_ops.cpp:421-428 (also jvp_SoftmaxRow, autodiff_jvp_ops.cpp:411-420)."""
    y, gy = np.asarray(y, dt), np.asarray(gy, dt)
    dot = _rsum(y * gy)
    if mut == 6:
        return y * gy - dot
    return y * (gy - dot)


def logsumexp_fwd(z, dt=np.float32, mut=0):
    """reduction.cpp:54-66.  Returns y keepdim ([..., 1])."""
    z = np.asarray(z, dt)
    m = _rmax(z)
    s = _rsum(np.exp(z - m))
    return np.log(s) if mut == 7 else np.log(s) + m


def _softmax_recomputed(z, dt, mut=0):
    m = _rmax(z)
    e = np.exp(z - m)
    return e if mut == 8 else e / _rsum(e)


def logsumexp_bwd(z, gy, dt=np.float32, mut=0):
    """autodiff_vjp_ops.cpp:430-440: gy ([..., 1]) * softmax(z), softmax recomputed."""
    z, gy = np.asarray(z, dt), np.asarray(gy, dt)
    return gy * _softmax_recomputed(z, dt, mut)


def logsumexp_jvp(z, tz, dt=np.float32, mut=0):
    """autodiff_jvp_ops.cpp:421-434: reduce_sum(softmax(z) * tz), keepdim."""
    z, tz = np.asarray(z, dt), np.asarray(tz, dt)
    return _rsum(_softmax_recomputed(z, dt, mut) * tz)


# ---- RMSNorm forward-mode product ---------------------------------------------------

def rmsnorm_jvp(x, gamma, tx, tgamma=None, eps=1e-5, dt=np.float32, mut=0):
    """Tangent of y = rms(x) * gamma along (tx, tgamma).

    rms node (normalization.cpp:23-35): r = 1/sqrt(mean(x*x) + eps), y = x*r;
    its tangent, corrected from autodiff_jvp_ops.cpp:366-379:
        dot = reduce_sum(tx * y);  ty = (tx * r) - (y * dot * r) / D
    then jvp_Mul for the gamma node: (ty * gamma) + (y * tgamma).
    gamma None: the rms node alone.
    """
    x, tx = np.asarray(x, dt), np.asarray(tx, dt)
    D = x.shape[-1]
    ms = _rmean(x * x)
    r = dt(1.0) / np.sqrt(ms + dt(eps))
    y = x * r
    dot = _rsum(tx * y)
    if mut == 9:  # the reference's rule as written: divides by tape[0] = r
        t = (tx / r) - (y * dot / (r * dt(D)))
    else:
        t = (tx * r) - (y * dot * r) / dt(D)
    if gamma is None:
        return t
    g = np.asarray(gamma, dt).reshape((1,) * (x.ndim - 1) + (D,))
    out = t * g
    if tgamma is not None and mut != 10:
        out = out + y * np.asarray(tgamma, dt).reshape(g.shape)
    return out


# ---- bf16 storage wrappers ----------------------------------------------------------
# Decode bf16 bit patterns to float32, run the float32 restatement, round the
# stored outputs to bf16 (per-row statistics stay float32).

def _dec(a):
    return None if a is None else bf16_decode(a)


def layernorm_fwd_bf16(x_bits, eps=1e-5):
    y, mean, var = layernorm_fwd(_dec(x_bits), eps)
    return bf16_encode(y), mean, var


def layernorm_bwd_bf16(x_bits, mean, var, gy_bits, eps=1e-5):
    return bf16_encode(layernorm_bwd(_dec(x_bits), mean, var, _dec(gy_bits), eps))


def softmax_fwd_bf16(z_bits):
    return bf16_encode(softmax_fwd(_dec(z_bits)))


def softmax_bwd_bf16(y_bits, gy_bits):
    return bf16_encode(softmax_bwd(_dec(y_bits), _dec(gy_bits)))


def logsumexp_fwd_bf16(z_bits):
    return bf16_encode(logsumexp_fwd(_dec(z_bits)))


def logsumexp_bwd_bf16(z_bits, gy_bits):
    return bf16_encode(logsumexp_bwd(_dec(z_bits), _dec(gy_bits)))


def logsumexp_jvp_bf16(z_bits, tz_bits):
    return bf16_encode(logsumexp_jvp(_dec(z_bits), _dec(tz_bits)))


def rmsnorm_jvp_bf16(x_bits, gamma_bits, tx_bits, tgamma_bits=None, eps=1e-5):
    return bf16_encode(rmsnorm_jvp(_dec(x_bits), _dec(gamma_bits), _dec(tx_bits),
                                   _dec(tgamma_bits), eps))


# ---- broadcast multiply ------------------------------------------------------------

def reduce_for_broadcast(g, target_shape, mut=0):
    """autodiff_vjp_ops.cpp:15-35: sum g over the axes where the target, aligned
    at the trailing axis, is missing or has extent 1 (and g's extent is not),
    keeping those axes, then reshape to the target.  Summed in float64."""
    target_shape = tuple(target_shape)
    if g.shape == target_shape:
        return g
    gnd, tnd = g.ndim, len(target_shape)
    axes = []
    for i in range(gnd):
        t = i + tnd - gnd if mut != 12 else i
        if t < 0 or t >= tnd:
            axes.append(i)
        elif target_shape[t] == 1 and g.shape[i] > 1 and mut != 11:
            axes.append(i)
    out = np.sum(g, axis=tuple(axes), keepdims=True, dtype=np.float64) if axes else g
    return out.reshape(target_shape)


def mul_bcast_fwd(a, b, dt=np.float32):
    """mul_nodeops (arithmetic.cpp:31-39): a * b with numpy broadcasting, one rounding."""
    return np.multiply(a.astype(dt), b.astype(dt), dtype=dt)


def mul_bcast_vjp(gy, a, b, mut=0):
    """vjp_Mul (autodiff_vjp_ops.cpp:54-59) in float64: (dA, dB), each
    reduce_for_broadcast(gy * other, operand).  Products of float32 or bf16
    values are exact in float64; the caller rounds (to storage for an operand
    of the output's shape, to float32 for a broadcast one)."""
    g = gy.astype(np.float64)
    da = reduce_for_broadcast(g * b.astype(np.float64), a.shape, mut)
    db = reduce_for_broadcast(g * a.astype(np.float64), b.shape, mut)
    return da, db


def mul_bcast_vjp_bf16(gy_bits, a_bits, b_bits, mut=0):
    """The same on bf16 storage: a gradient with the output's shape is the
    product rounded to bf16 bits; a broadcast operand's is a float32 sum."""
    gy, a, b = _dec(gy_bits), _dec(a_bits), _dec(b_bits)
    da, db = mul_bcast_vjp(gy, a, b, mut)
    out_ndim = gy.ndim

    def finish(d, shape):
        aligned = (1,) * (out_ndim - len(shape)) + tuple(shape)
        if aligned == gy.shape:
            return bf16_encode(d.astype(np.float32))
        return d.astype(np.float32)
    return finish(da, a.shape), finish(db, b.shape)

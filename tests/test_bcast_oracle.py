"""Pins of the broadcast-multiply oracle (oracle/rowops.py: mul_bcast_fwd,
reduce_for_broadcast, mul_bcast_vjp), on the CPU.

The oracle restates reduce_for_broadcast (autodiff_vjp_ops.cpp:15-35) as a sum
over axes.  It is checked against formulations that share none of that axis
logic:
  - a brute-force scatter-add over every output position (each position adds
    gy * other into the operand entry it was broadcast from, the index found by
    taking the output index modulo 1 on the operand's extent-1 axes);
  - the adjoint identity <gy, a * b> = <dA, a> = <dB, b>, which holds for the
    VJP of a bilinear product whatever the broadcast;
  - special cases: equal shapes (no reduction), a scalar operand (the whole
    sum), the forward against numpy's broadcasting multiply.
test_planted_mistakes_are_caught shows that each mistake the oracle can be
built with (mut 11: extent-1 axes not summed; mut 12: shapes aligned at the
leading axis) fails one of these checks.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest

import oracle
from oracle import rowops as ro

# (a shape, b shape): every broadcast form the graph layer can meet
PAIRS = [
    ((3, 4), (3, 4)),           # equal
    ((3, 4), (4,)),             # row vector, missing axis
    ((3, 4), (1, 4)),           # row vector, extent-1 axis
    ((3, 1), (1, 4)),           # outer product: both reduced
    ((2, 3, 4), (2, 1, 4)),     # middle axis
    ((2, 3, 4), (3, 1)),        # missing leading axis and trailing extent 1
    ((1,), (2, 3)),             # scalar-like
    ((), (2, 3)),               # 0-d scalar
    ((2, 1, 3, 1), (1, 4, 1, 5)),
    ((5, 1, 1), (1, 1)),
]


def _rng(seed):
    return np.random.default_rng(seed)


def _inputs(a_shape, b_shape, seed):
    g = _rng(seed)
    a = g.standard_normal(a_shape)
    b = g.standard_normal(b_shape)
    out = np.broadcast_shapes(a_shape, b_shape)
    gy = g.standard_normal(out)
    return gy, a, b


def _brute_force(gy, a, b):
    """Scatter-add: each output position adds gy * b into the entry of a it read
    (and gy * a into b's)."""
    out = gy.shape
    nd = len(out)
    pa = (1,) * (nd - a.ndim) + a.shape
    pb = (1,) * (nd - b.ndim) + b.shape
    A = a.reshape(pa)
    B = b.reshape(pb)
    da = np.zeros(pa)
    db = np.zeros(pb)
    for idx in itertools.product(*[range(n) for n in out]):
        ia = tuple(i if e != 1 else 0 for i, e in zip(idx, pa))
        ib = tuple(i if e != 1 else 0 for i, e in zip(idx, pb))
        da[ia] += gy[idx] * B[ib]
        db[ib] += gy[idx] * A[ia]
    return da.reshape(a.shape), db.reshape(b.shape)


def _pins(mut):
    """The pins as (name, ok) pairs for the oracle built with `mut`."""
    res = []
    for k, (sa, sb) in enumerate(PAIRS):
        gy, a, b = _inputs(sa, sb, 100 + k)
        try:
            da, db = ro.mul_bcast_vjp(gy, a, b, mut=mut)
        except ValueError:  # a mistaken reduction that cannot even reshape
            res.append((f"brute force {sa} {sb}", False))
            continue
        ra, rb = _brute_force(gy, a, b)
        res.append((f"brute force {sa} {sb}",
                    da.shape == a.shape and db.shape == b.shape and
                    np.allclose(da, ra, rtol=1e-12, atol=1e-12) and
                    np.allclose(db, rb, rtol=1e-12, atol=1e-12)))
        lhs = float(np.sum(gy * (a * b)))
        res.append((f"adjoint {sa} {sb}",
                    np.isclose(float(np.sum(da * a)), lhs, rtol=1e-10, atol=1e-10) and
                    np.isclose(float(np.sum(db * b)), lhs, rtol=1e-10, atol=1e-10)))
    return res


def test_oracle_passes_its_pins():
    bad = [name for name, ok in _pins(0) if not ok]
    assert not bad, bad


@pytest.mark.parametrize("mut", [11, 12])
def test_planted_mistakes_are_caught(mut):
    assert any(not ok for _, ok in _pins(mut)), f"mutation {mut} passed every pin"


def test_special_cases():
    g = _rng(7)
    a = g.standard_normal((4, 5))
    b = g.standard_normal((4, 5))
    gy = g.standard_normal((4, 5))
    da, db = ro.mul_bcast_vjp(gy, a, b)
    assert np.array_equal(da, gy * b) and np.array_equal(db, gy * a)  # no reduction
    s = np.array(1.5)
    da, ds = ro.mul_bcast_vjp(gy, a, s)
    assert ds.shape == () and np.isclose(float(ds), float(np.sum(gy * a)), rtol=1e-13)
    assert np.array_equal(da, gy * 1.5)


def test_forward_is_numpy_broadcasting():
    for k, (sa, sb) in enumerate(PAIRS):
        _, a, b = _inputs(sa, sb, 200 + k)
        a32, b32 = a.astype(np.float32), b.astype(np.float32)
        y = ro.mul_bcast_fwd(a32, b32)
        assert y.dtype == np.float32 and y.shape == np.broadcast_shapes(sa, sb)
        assert np.array_equal(y, a32 * b32)


def test_bf16_wrapper_rounds_full_gradients_to_storage():
    gy, a, b = _inputs((3, 4), (1, 4), 9)
    enc = oracle.bf16_encode
    da, db = ro.mul_bcast_vjp_bf16(enc(gy.astype(np.float32)), enc(a.astype(np.float32)),
                                   enc(b.astype(np.float32)))
    assert da.dtype == np.uint16 and da.shape == (3, 4)      # full: bf16 bits
    assert db.dtype == np.float32 and db.shape == (1, 4)     # broadcast: float32 sum

"""Parity of the general broadcast multiply (agk_mul_bcast_fwd / _bwd) with the
pinned oracle (oracle/rowops.py: mul_bcast_fwd, mul_bcast_vjp).

Bars:
  - the forward and the gradient of an operand with the output's shape are one
    product (plus, when accumulating, one add) rounded to storage: bit-exact
    against the oracle's float32 arithmetic (bf16: rounded to bf16 bits);
  - the gradient of a broadcast operand is a float64 sum of exact products
    rounded to float32 once; the device sums in another order, so the result
    may differ in the last float32 place: relative error <= 2^-22 (two float32
    ulps) per element, against the oracle's float64 sum;
  - results are identical run to run.
Shapes cover every broadcast form (missing axes, extent-1 axes, both operands
reduced, 0-d scalars, long reductions that take the 256-lane reduction, empty
outputs) in fp32 and bf16.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import cgadimpl_amd as agk
from gpu_util import to_dev, to_host
from oracle import rowops as ro
from tolerances import TOL_F32

pytestmark = pytest.mark.gpu

PAIRS = [
    ((3, 4), (3, 4)),
    ((3, 4), (4,)),
    ((7, 1), (1, 9)),
    ((2, 3, 4), (2, 1, 4)),
    ((2, 3, 4), (3, 1)),
    ((1,), (5, 6)),
    ((), (5, 6)),
    ((2, 1, 3, 1), (1, 4, 1, 5)),
    ((4, 33, 130), (4, 1, 130)),
    ((6, 700, 3), (1, 700, 1)),        # long sums for b (256-lane reduction)
    ((1, 1), (5000, 3)),               # a summed over 15000 products
    ((64, 1, 96), (64, 40, 1)),
    ((8, 64, 96), (1, 1, 96)),         # column sums whose quarters cross outer positions
    ((6, 5, 4, 32), (6, 1, 1, 32)),    # two reduced axes between kept ones
    ((4, 33, 128), (4, 1, 128)),       # 16-byte forward in bf16 too
]
REL = 2.0 ** -22


def _operands(sa, sb, seed, dtype):
    g = np.random.default_rng(seed)
    out = np.broadcast_shapes(sa, sb)
    a = g.standard_normal(sa).astype(np.float32)
    b = g.standard_normal(sb).astype(np.float32)
    gy = g.standard_normal(out).astype(np.float32)
    if dtype == "bf16":  # (bf16_encode makes a 0-d array 1-d: reshape back)
        return tuple(oracle.bf16_encode(t).reshape(t.shape) for t in (gy, a, b))
    return gy, a, b


def _f32(t):  # (bf16_decode makes a 0-d array 1-d: reshape back)
    return oracle.bf16_decode(t).reshape(t.shape) if t.dtype == np.uint16 else t


def _check_grad(got, ref64, full, dtype, what):
    if full:  # product rounded to storage
        want = ref64.astype(np.float32)
        if dtype == "bf16":
            want = oracle.bf16_encode(want)
        assert got.dtype == want.dtype and got.shape == want.shape, what
        assert np.array_equal(got, want), what
    else:
        assert got.dtype == np.float32 and got.shape == ref64.shape, what
        err = np.abs(got.astype(np.float64) - ref64)
        assert np.all(err <= REL * np.abs(ref64) + 1e-30), (what, float(err.max()))


def _is_full(shape, out):
    return (1,) * (len(out) - len(shape)) + tuple(shape) == tuple(out)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("sa,sb", PAIRS, ids=lambda v: str(v))
def test_forward_and_vjp_match_oracle(cuda, sa, sb, dtype):
    gy, a, b = _operands(sa, sb, 11, dtype)
    out = np.broadcast_shapes(sa, sb)
    # (np.ascontiguousarray, inside to_dev, makes a 0-d array 1-d: reshape back)
    ad, bd, gyd = to_dev(a, cuda).reshape(sa), to_dev(b, cuda).reshape(sb), to_dev(gy, cuda)
    print(f"bcast {dtype} a{sa} b{sb}", flush=True)
    assert agk.mul_bcast_shape(sa, sb) == tuple(out)
    y = to_host(agk.mul_bcast_fwd(ad, bd))
    want = ro.mul_bcast_fwd(_f32(a), _f32(b))
    if dtype == "bf16":
        want = oracle.bf16_encode(want)
    assert y.shape == tuple(out) and np.array_equal(y, want)
    da, db = agk.mul_bcast_bwd(gyd, ad, bd)
    ra, rb = ro.mul_bcast_vjp(_f32(gy), _f32(a), _f32(b))
    _check_grad(to_host(da), ra, _is_full(sa, out), dtype, "da")
    _check_grad(to_host(db), rb, _is_full(sb, out), dtype, "db")
    # run to run
    da2, db2 = agk.mul_bcast_bwd(gyd, ad, bd)
    assert np.array_equal(to_host(da2), to_host(da)) and np.array_equal(to_host(db2), to_host(db))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_accumulation(cuda, dtype):
    sa, sb = (4, 33, 130), (4, 1, 130)
    gy, a, b = _operands(sa, sb, 12, dtype)
    ad, bd, gyd = to_dev(a, cuda), to_dev(b, cuda), to_dev(gy, cuda)
    import torch
    da0 = to_dev(_operands(sa, sa, 13, dtype)[1], cuda)            # prior gradient of a
    db0 = torch.from_numpy(np.random.default_rng(14).standard_normal(sb).astype(np.float32)).to(cuda)
    pre_a, pre_b = to_host(da0).copy(), to_host(db0).copy()
    da, db = agk.mul_bcast_bwd(gyd, ad, bd, da=da0, db=db0, accumulate=True)
    ra, rb = ro.mul_bcast_vjp(_f32(gy), _f32(a), _f32(b))
    # full operand: old + product, each rounded to storage (float32 arithmetic)
    prod = ra.astype(np.float32)
    if dtype == "bf16":
        prod = _f32(oracle.bf16_encode(prod))
        want = oracle.bf16_encode(_f32(pre_a) + prod)
    else:
        want = pre_a + prod
    assert np.array_equal(to_host(da), want)
    # broadcast operand: old + float64 sum, rounded once
    ref = pre_b.astype(np.float64) + rb
    got = to_host(db).astype(np.float64)
    assert np.all(np.abs(got - ref) <= REL * np.abs(ref) + 1e-30)
    # forward accumulation: y += a * b
    y0 = to_dev(_operands(sa, sa, 15, dtype)[1], cuda)
    pre_y = to_host(y0).copy()
    y = to_host(agk.mul_bcast_fwd(ad, bd, y=y0, accumulate=True))
    p = ro.mul_bcast_fwd(_f32(a), _f32(b))
    if dtype == "bf16":
        want = oracle.bf16_encode(_f32(pre_y) + _f32(oracle.bf16_encode(p)))
    else:
        want = pre_y + p
    assert np.array_equal(y, want)


def test_empty_output_gives_zero_gradients(cuda):
    """a [3, 0, 4] * b [3, 1, 4]: the output is empty and b's gradient is an
    empty sum, zeros.  (The reference's reduce_for_broadcast sums only axes
    whose extent is above 1, so it cannot reshape this case; the kernel gives
    the mathematical answer.)"""
    import torch
    a = torch.zeros(3, 0, 4, device=cuda)
    b = torch.ones(3, 1, 4, device=cuda)
    gy = torch.zeros(3, 0, 4, device=cuda)
    assert agk.mul_bcast_fwd(a, b).shape == (3, 0, 4)
    db0 = torch.full((3, 1, 4), 7.0, device=cuda)
    da, db = agk.mul_bcast_bwd(gy, a, b, db=db0)
    assert da.shape == (3, 0, 4) and db.dtype == torch.float32
    assert torch.count_nonzero(db).item() == 0
    db1 = torch.full((3, 1, 4), 7.0, device=cuda)
    _, db = agk.mul_bcast_bwd(gy, a, b, db=db1, want_da=False, accumulate=True)
    assert torch.all(db == 7.0).item()


def test_rejects_incompatible_shapes(cuda):
    import torch
    a = torch.zeros(3, 4, device=cuda)
    b = torch.zeros(2, 4, device=cuda)
    with pytest.raises(RuntimeError, match="AGK_EINVAL"):
        agk.mul_bcast_fwd(a, b, y=torch.zeros(3, 4, device=cuda))
    with pytest.raises(RuntimeError, match="AGK_EINVAL"):
        agk.mul_bcast_shape((2, 3, 4, 5, 6, 7, 8, 9, 10), (1,))   # more than 8 axes


def test_row_vector_cases_agree_with_the_row_kernels(cuda):
    """The row-vector broadcast has its own kernels (agk_mul_rowbcast_*); the
    general path must give the same bits for it."""
    gy, a, b = _operands((300, 257), (257,), 21, "f32")
    ad, bd, gyd = to_dev(a, cuda), to_dev(b, cuda), to_dev(gy, cuda)
    y1 = to_host(agk.mul_bcast_fwd(ad, bd))
    y2 = to_host(agk.mul_rowbcast_fwd(ad, bd))
    assert np.array_equal(y1, y2)
    da1, db1 = agk.mul_bcast_bwd(gyd, ad, bd)
    da2, db2 = agk.mul_rowbcast_bwd(gyd, ad, bd)
    assert np.array_equal(to_host(da1), to_host(da2))
    r = ro.mul_bcast_vjp(gy, a, b)[1]
    # the general kernel: two float32 ulps of the float64 sum; the row kernel
    # sums float32 partial rows first and is held to its own dgamma bar
    # (1e-5 of the largest column sum, tests/tolerances.py)
    g1, g2 = to_host(db1).astype(np.float64), to_host(db2).astype(np.float64)
    assert np.all(np.abs(g1 - r) <= REL * np.abs(r) + 1e-30)
    assert np.max(np.abs(g2 - r)) <= TOL_F32 * np.max(np.abs(r))

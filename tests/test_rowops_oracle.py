"""Pins of the row-op oracle (oracle/rowops.py), on the CPU.

Each restated function is checked against something that does not share its
formula:
  - a library routine (torch.nn.functional.layer_norm, scipy.special.softmax
    and logsumexp, torch autograd and torch.func.jvp) in float64;
  - central finite differences of the forward, in float64;
  - the adjoint identity <dy, J t> = <J^T dy, t> between a forward-mode
    product and a backward product that is pinned on its own (for the
    RMSNorm JVP: the fp64 closed form of the RMSNorm VJP in the C oracle);
  - invariants (softmax rows sum to 1, sum of a LayerNorm or softmax VJP
    row is 0, the log-sum-exp VJP row sums to dy, shift invariance) and
    special cases (constant rows, one-element rows, overflow-sized inputs).
test_planted_mistakes_are_caught shows that each mistake the oracle can be
built with (its `mut` argument) fails at least one of these checks, and
test_reference_jvp_rule_is_wrong records that the reference's own RMSNorm
forward-mode rule fails the finite-difference check.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import rowops as ro

torch = pytest.importorskip("torch")
special = pytest.importorskip("scipy.special")

F64 = np.float64


def _rng(seed):
    return np.random.default_rng(seed)


def _inputs(seed, shape=(6, 11), scale=1.0):
    g = _rng(seed)
    return g.standard_normal(shape) * scale, g.standard_normal(shape)


def _fd_vjp(f, x, gy, h=1e-6):
    """Gradient of sum(gy * f(x)) by central differences (float64)."""
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        xp, xm = x.copy(), x.copy()
        xp[i] += h
        xm[i] -= h
        g[i] = (np.sum(gy * f(xp)) - np.sum(gy * f(xm))) / (2 * h)
    return g


def _fd_dir(f, x, t, h=1e-6):
    """Directional derivative (f(x + h t) - f(x - h t)) / 2h (float64)."""
    return (f(x + h * t) - f(x - h * t)) / (2 * h)


def _rel(a, b):
    a, b = np.asarray(a, F64), np.asarray(b, F64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


# ---- the checks (each returns True when the oracle passes it) ---------------------

def ln_fwd_checks(mut=0):
    x, _ = _inputs(1)
    eps = 1e-2  # large enough that a dropped eps is visible
    y, mean, var = ro.layernorm_fwd(x, eps, dt=F64, mut=mut)
    want = torch.nn.functional.layer_norm(torch.from_numpy(x), (x.shape[-1],), eps=eps).numpy()
    ok_lib = _rel(y, want) < 1e-12
    ok_stats = _rel(mean, x.mean(-1, keepdims=True)) < 1e-14 and \
        _rel(var, x.var(-1, keepdims=True)) < 1e-12
    yc, _, vc = ro.layernorm_fwd(np.full((2, 7), 3.25, np.float32), mut=mut)
    ok_const = np.all(yc == 0) and np.all(vc == 0)
    return ok_lib and ok_stats and ok_const


def ln_bwd_checks(mut=0):
    x, gy = _inputs(2)
    eps = 1e-5
    _, mean, var = ro.layernorm_fwd(x, eps, dt=F64)
    dx = ro.layernorm_bwd(x, mean, var, gy, eps, dt=F64, mut=mut)
    fd = _fd_vjp(lambda v: ro.layernorm_fwd(v, eps, dt=F64)[0], x, gy)
    xt = torch.from_numpy(x).requires_grad_(True)
    torch.nn.functional.layer_norm(xt, (x.shape[-1],), eps=eps).backward(torch.from_numpy(gy))
    ok_fd = _rel(dx, fd) < 1e-6
    ok_lib = _rel(dx, xt.grad.numpy()) < 1e-10
    ok_sum = np.max(np.abs(dx.sum(-1))) < 1e-10 * np.max(np.abs(dx))
    return ok_fd and ok_lib and ok_sum


def sm_fwd_checks(mut=0):
    z, _ = _inputs(3, scale=3.0)
    y = ro.softmax_fwd(z, dt=F64, mut=mut)
    ok_lib = _rel(y, special.softmax(z, axis=-1)) < 1e-14
    ok_sum = np.max(np.abs(y.sum(-1) - 1)) < 1e-14
    ok_shift = _rel(ro.softmax_fwd(z + 17.5, dt=F64, mut=mut), y) < 1e-12
    big = ro.softmax_fwd(np.array([[1000.0, 1000.0, -np.inf]], np.float32), mut=mut)
    ok_big = np.array_equal(big, np.array([[0.5, 0.5, 0.0]], np.float32))
    return ok_lib and ok_sum and ok_shift and ok_big


def sm_bwd_checks(mut=0):
    z, gy = _inputs(4, scale=2.0)
    y = ro.softmax_fwd(z, dt=F64)
    dz = ro.softmax_bwd(y, gy, dt=F64, mut=mut)
    fd = _fd_vjp(lambda v: ro.softmax_fwd(v, dt=F64), z, gy)
    zt = torch.from_numpy(z).requires_grad_(True)
    torch.softmax(zt, -1).backward(torch.from_numpy(gy))
    return (_rel(dz, fd) < 1e-6 and _rel(dz, zt.grad.numpy()) < 1e-12 and
            np.max(np.abs(dz.sum(-1))) < 1e-12)


def lse_fwd_checks(mut=0):
    z, _ = _inputs(5, scale=4.0)
    y = ro.logsumexp_fwd(z, dt=F64, mut=mut)
    ok_lib = _rel(y, special.logsumexp(z, axis=-1, keepdims=True)) < 1e-14
    ok_shift = _rel(ro.logsumexp_fwd(z + 9.0, dt=F64, mut=mut), y + 9.0) < 1e-13
    one = ro.logsumexp_fwd(np.array([[2.5], [-7.0]], np.float32), mut=mut)
    ok_one = np.array_equal(one, np.array([[2.5], [-7.0]], np.float32))
    big = ro.logsumexp_fwd(np.array([[1000.0, 1000.0]]), dt=F64, mut=mut)
    ok_big = abs(big[0, 0] - (1000.0 + np.log(2.0))) < 1e-12
    return ok_lib and ok_shift and ok_one and ok_big


def lse_bwd_checks(mut=0):
    z, _ = _inputs(6, scale=2.0)
    gy = _rng(7).standard_normal((z.shape[0], 1))
    dz = ro.logsumexp_bwd(z, gy, dt=F64, mut=mut)
    fd = _fd_vjp(lambda v: ro.logsumexp_fwd(v, dt=F64), z, gy)
    zt = torch.from_numpy(z).requires_grad_(True)
    torch.logsumexp(zt, -1, keepdim=True).backward(torch.from_numpy(gy))
    return (_rel(dz, fd) < 1e-6 and _rel(dz, zt.grad.numpy()) < 1e-12 and
            _rel(dz.sum(-1, keepdims=True), gy) < 1e-12)


def lse_jvp_checks(mut=0):
    z, tz = _inputs(8, scale=2.0)
    ty = ro.logsumexp_jvp(z, tz, dt=F64, mut=mut)
    fd = _fd_dir(lambda v: ro.logsumexp_fwd(v, dt=F64), z, tz)
    gy = _rng(9).standard_normal((z.shape[0], 1))
    lhs = np.sum(gy * ty)
    rhs = np.sum(ro.logsumexp_bwd(z, gy, dt=F64) * tz)
    return _rel(ty, fd) < 1e-6 and abs(lhs - rhs) < 1e-12 * max(1.0, abs(rhs))


def _rms_layer_f64(x, g, eps):
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * r * g


def rms_jvp_checks(mut=0):
    g = _rng(10)
    x = g.standard_normal((5, 12))
    gam = g.uniform(0.5, 1.5, 12)
    tx = g.standard_normal((5, 12))
    tg = g.standard_normal(12)
    eps = 1e-5
    ty = ro.rmsnorm_jvp(x, gam, tx, tg, eps, dt=F64, mut=mut)
    fd = (_rms_layer_f64(x + 1e-6 * tx, gam + 1e-6 * tg, eps) -
          _rms_layer_f64(x - 1e-6 * tx, gam - 1e-6 * tg, eps)) / 2e-6
    ok_fd = _rel(ty, fd) < 1e-6
    # adjoint identity against the fp64 closed-form VJP of the C oracle
    dy = g.standard_normal((5, 12))
    _, _, dx, dgam = oracle.truth(x, gam, dy, eps)
    lhs = np.sum(dy * ty)
    rhs = np.sum(dx * tx) + np.sum(dgam * tg)
    ok_adj = abs(lhs - rhs) < 1e-10 * max(1.0, abs(rhs))
    # torch forward-mode product
    fwd = lambda a, b: a * torch.rsqrt(torch.mean(a * a, -1, keepdim=True) + eps) * b
    _, tj = torch.func.jvp(fwd, (torch.from_numpy(x), torch.from_numpy(gam)),
                           (torch.from_numpy(tx), torch.from_numpy(tg)))
    ok_lib = _rel(ty, tj.numpy()) < 1e-12
    # the unscaled node (ag::rms): tangent of x * r alone
    t0 = ro.rmsnorm_jvp(x, None, tx, None, eps, dt=F64, mut=mut)
    fd0 = _fd_dir(lambda v: _rms_layer_f64(v, 1.0, eps), x, tx)
    ok_node = _rel(t0, fd0) < 1e-6
    return ok_fd and ok_adj and ok_lib and ok_node


CHECKS = {
    "layernorm_fwd": ln_fwd_checks, "layernorm_bwd": ln_bwd_checks,
    "softmax_fwd": sm_fwd_checks, "softmax_bwd": sm_bwd_checks,
    "logsumexp_fwd": lse_fwd_checks, "logsumexp_bwd": lse_bwd_checks,
    "logsumexp_jvp": lse_jvp_checks, "rmsnorm_jvp": rms_jvp_checks,
}


@pytest.mark.parametrize("name", sorted(CHECKS))
def test_oracle_passes_its_pins(name):
    assert CHECKS[name](0)


@pytest.mark.parametrize("mut", range(1, 11))
def test_planted_mistakes_are_caught(mut):
    failed = [name for name, check in CHECKS.items() if not check(mut)]
    assert failed, f"mutation {mut} passed every check"


def test_reference_jvp_rule_is_wrong():
    """autodiff_jvp_ops.cpp:366-379 divides by tape[0] = 1/rms: it fails the FD check."""
    assert not rms_jvp_checks(9)


def test_layernorm_and_softmax_jacobians_are_symmetric():
    """The VJP rule applied to a tangent gives the JVP (used for forward mode)."""
    x, t = _inputs(11)
    _, mean, var = ro.layernorm_fwd(x, 1e-5, dt=F64)
    fd = _fd_dir(lambda v: ro.layernorm_fwd(v, 1e-5, dt=F64)[0], x, t)
    assert _rel(ro.layernorm_bwd(x, mean, var, t, 1e-5, dt=F64), fd) < 1e-6
    y = ro.softmax_fwd(x, dt=F64)
    fd = _fd_dir(lambda v: ro.softmax_fwd(v, dt=F64), x, t)
    assert _rel(ro.softmax_bwd(y, t, dt=F64), fd) < 1e-6


def test_float32_path_tracks_float64():
    x, t = _inputs(12, shape=(16, 300), scale=2.0)
    for f in (lambda d: ro.layernorm_fwd(x, 1e-5, dt=d)[0],
              lambda d: ro.softmax_fwd(x, dt=d),
              lambda d: ro.logsumexp_fwd(x, dt=d),
              lambda d: ro.rmsnorm_jvp(x, None, t, None, 1e-5, dt=d)):
        assert _rel(f(np.float32), f(F64)) < 1e-5


def test_bf16_wrappers_round_outputs_once():
    x, t = _inputs(13, shape=(8, 64))
    xb = oracle.bf16_encode(x.astype(np.float32))
    y = ro.softmax_fwd_bf16(xb)
    assert y.dtype == np.uint16
    want = oracle.bf16_encode(ro.softmax_fwd(oracle.bf16_decode(xb)))
    assert np.array_equal(y, want)
    ref = special.softmax(oracle.bf16_decode(xb).astype(F64), axis=-1)
    assert _rel(oracle.bf16_decode(y), ref) < 2.0 ** -8

"""Checks that pin the CPU oracle to something other than itself.

Each check returns a list of failure strings (empty = pass), so the same
suite can run against the real oracle (must pass) and against builds with a
planted mistake (each must fail at least one check).  What pins what:

  golden       torch.nn.functional.rms_norm + autograd in float64 on fixed
               inputs (tests/golden/rmsnorm_golden.json): y, inv_rms, dx, dgamma
  fd_dx        central differences of the oracle's own fp32 forward, the
               reference's numerical-gradient pattern
               (cgadimpl/Tests/test_core_ops_gpu.cpp:38-84: h=1e-4, tol 1e-3;
               here h=1e-3 with the loss accumulated in fp64)
  fd_dgamma    the same for gamma
  fd_truth     central differences of the fp64 closed form (h=1e-6, tol 1e-7)
  invariant    sum_j x_j dx_j = dot * eps * r^3 per row (dot = sum g x)
  special      zero row: y = 0, r = eps^-1/2; constant row c:
               y = gamma c / sqrt(c^2 + eps); width 1: dx = g eps r^3;
               scale invariance y(1000 x) ~ y(x)
  dgamma_ones  dy = 1, no gamma: dgamma = column sums of the forward output
  permutation  permuting rows permutes y and dx and leaves dgamma unchanged
  accumulate   accumulate=1 adds onto existing gradients
  linear       the RMSNorm + linear layer: y = h I = h for an identity W; central
               differences of sum(y * dy) with respect to h and W give dh and dW;
               the layer's dx equals the RMSNorm VJP of dh = dy W^T
"""
from __future__ import annotations

import json
import os

import numpy as np

import oracle
from tolerances import TOL_F32, row_rel_err, vec_rel_err

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "rmsnorm_golden.json")


def golden_cases():
    with open(GOLDEN) as fh:
        return json.load(fh)["cases"]


def _arr(case, key):
    v = case[key]
    if v is None:
        return None
    a = np.asarray(v, dtype=np.float64)
    if key in ("x", "dy", "y", "dx"):
        a = a.reshape(case["shape"])
    elif key == "inv_rms":
        a = a.reshape(case["shape"][:-1])
    return a


def check_golden(mutation: int = 0):
    fails = []
    for c in golden_cases():
        x = _arr(c, "x").astype(np.float32)
        g = _arr(c, "gamma")
        g = None if g is None else g.astype(np.float32)
        dy = _arr(c, "dy").astype(np.float32)
        eps = c["eps"]
        y, inv = oracle.fwd(x, g, eps, mutation=mutation)
        dx, dg = oracle.bwd(x, g, inv, dy, mutation=mutation)
        errs = {
            "y": row_rel_err(y, _arr(c, "y")),
            "inv_rms": vec_rel_err(inv, _arr(c, "inv_rms")),
            "dx": row_rel_err(dx, _arr(c, "dx")),
        }
        if c["dgamma"] is not None:
            errs["dgamma"] = vec_rel_err(dg, _arr(c, "dgamma"))
        # fp64 closed form against the same fixture (tight)
        ty, tinv, tdx, tdg = oracle.truth(x, g, dy, eps, mutation=mutation)
        terrs = {"y": row_rel_err(ty, _arr(c, "y")), "dx": row_rel_err(tdx, _arr(c, "dx"))}
        if c["dgamma"] is not None:
            terrs["dgamma"] = vec_rel_err(tdg, _arr(c, "dgamma"))
        for k, e in errs.items():
            if not e <= TOL_F32:
                fails.append(f"golden {c['name']} oracle {k}: rel err {e:.3g}")
        for k, e in terrs.items():
            if not e <= 1e-12:
                fails.append(f"golden {c['name']} truth {k}: rel err {e:.3g}")
    return fails


def _loss(x, g, dy, eps, mutation):
    y, _ = oracle.fwd(x, g, eps, mutation=mutation)
    return float(np.sum(y.astype(np.float64) * dy.astype(np.float64)))


def check_fd(mutation: int = 0):
    """Central differences of the fp32 oracle forward vs its backward."""
    fails = []
    rng = np.random.default_rng(3)
    for shape, eps, with_gamma in (((4, 10), 1e-5, False), ((3, 12), 1e-6, True),
                                   ((2, 9), 0.5, True)):
        x = rng.standard_normal(shape).astype(np.float32)
        g = rng.uniform(0.5, 1.5, shape[-1]).astype(np.float32) if with_gamma else None
        dy = rng.standard_normal(shape).astype(np.float32)
        _, inv = oracle.fwd(x, g, eps, mutation=mutation)
        dx, dg = oracle.bwd(x, g, inv, dy, mutation=mutation)
        h = 1e-3
        num = np.zeros(x.size)
        xf = x.ravel()
        for i in range(x.size):
            xp = xf.copy(); xp[i] += h
            xm = xf.copy(); xm[i] -= h
            num[i] = (_loss(xp.reshape(shape), g, dy, eps, mutation)
                      - _loss(xm.reshape(shape), g, dy, eps, mutation)) / (
                          float(np.float32(xf[i] + h)) - float(np.float32(xf[i] - h)))
        e = np.max(np.abs(num - dx.ravel()))
        if not e <= 1e-3:
            fails.append(f"fd_dx {shape} eps={eps}: max|diff| {e:.3g}")
        if with_gamma:
            numg = np.zeros(shape[-1])
            for j in range(shape[-1]):
                gp = g.copy(); gp[j] += h
                gm = g.copy(); gm[j] -= h
                numg[j] = (_loss(x, gp, dy, eps, mutation) - _loss(x, gm, dy, eps, mutation)) / (
                    float(np.float32(g[j] + h)) - float(np.float32(g[j] - h)))
            e = np.max(np.abs(numg - dg))
            if not e <= 1e-3:
                fails.append(f"fd_dgamma {shape} eps={eps}: max|diff| {e:.3g}")
    return fails


def check_fd_truth(mutation: int = 0):
    fails = []
    rng = np.random.default_rng(11)
    shape, eps = (3, 7), 0.05
    x = rng.standard_normal(shape)
    g = rng.uniform(0.5, 1.5, shape[-1])
    dy = rng.standard_normal(shape)
    _, _, dx, dg = oracle.truth(x, g, dy, eps, mutation=mutation)

    def loss(xx, gg):
        y, _, _, _ = oracle.truth(xx, gg, None, eps, mutation=mutation)
        return float(np.sum(y * dy))

    h = 1e-6
    num = np.zeros(x.size)
    for i in range(x.size):
        xp = x.ravel().copy(); xp[i] += h
        xm = x.ravel().copy(); xm[i] -= h
        num[i] = (loss(xp.reshape(shape), g) - loss(xm.reshape(shape), g)) / (2 * h)
    if not np.max(np.abs(num - dx.ravel())) <= 1e-7:
        fails.append("fd_truth dx")
    numg = np.zeros(shape[-1])
    for j in range(shape[-1]):
        gp = g.copy(); gp[j] += h
        gm = g.copy(); gm[j] -= h
        numg[j] = (loss(x, gp) - loss(x, gm)) / (2 * h)
    if not np.max(np.abs(numg - dg)) <= 1e-7:
        fails.append("fd_truth dgamma")
    return fails


def check_invariant(mutation: int = 0):
    """sum_j x_j dx_j = dot * eps * r^3 (row-wise), dot = sum_j (dy_j gamma_j) x_j."""
    fails = []
    rng = np.random.default_rng(5)
    for shape, eps, scale in (((6, 33), 0.5, 1.0), ((4, 64), 1e-2, 0.1), ((3, 16), 1e-6, 1.0)):
        x = (scale * rng.standard_normal(shape)).astype(np.float32)
        g = rng.uniform(0.5, 1.5, shape[-1]).astype(np.float32)
        dy = rng.standard_normal(shape).astype(np.float32)
        _, inv = oracle.fwd(x, g, eps, mutation=mutation)
        dx, _ = oracle.bwd(x, g, inv, dy, mutation=mutation)
        x64, dx64 = x.astype(np.float64), dx.astype(np.float64)
        gy = dy.astype(np.float64) * g.astype(np.float64)
        dot = np.sum(gy * x64, axis=-1)
        ms = np.mean(x64 * x64, axis=-1)
        r = 1.0 / np.sqrt(ms + eps)
        lhs = np.sum(x64 * dx64, axis=-1)
        rhs = dot * eps * r ** 3
        scale_ref = r * np.sum(np.abs(gy * x64), axis=-1)
        err = np.max(np.abs(lhs - rhs) / scale_ref)
        if not err <= 1e-5:
            fails.append(f"invariant {shape} eps={eps}: {err:.3g}")
    return fails


def check_special(mutation: int = 0):
    fails = []
    D = 8
    g = np.linspace(0.5, 1.5, D).astype(np.float32)
    eps = 1e-5
    x = np.zeros((3, D), dtype=np.float32)
    x[1, :] = 2.0
    x[2, :] = -0.5
    y, inv = oracle.fwd(x, g, eps, mutation=mutation)
    if not np.all(y[0] == 0.0):
        fails.append("special zero row: y != 0")
    if not abs(inv[0] - np.float32(1.0) / np.sqrt(np.float32(eps))) <= 1e-6 * inv[0]:
        fails.append(f"special zero row: inv_rms {inv[0]}")
    for row, c in ((1, 2.0), (2, -0.5)):
        want = g.astype(np.float64) * c / np.sqrt(c * c + eps)
        if not np.max(np.abs(y[row] - want)) <= 1e-6 * np.max(np.abs(want)):
            fails.append(f"special constant row {c}")
    # width 1: y = gamma x / sqrt(x^2+eps), dx = dy gamma eps r^3
    x1 = np.array([[0.3], [-2.0], [1e-3]], dtype=np.float32)
    g1 = np.array([1.25], dtype=np.float32)
    dy1 = np.array([[1.0], [0.5], [-2.0]], dtype=np.float32)
    eps1 = 1e-2
    y1, inv1 = oracle.fwd(x1, g1, eps1, mutation=mutation)
    dx1, _ = oracle.bwd(x1, g1, inv1, dy1, mutation=mutation)
    xd = x1.astype(np.float64)
    r1 = 1.0 / np.sqrt(xd * xd + eps1)
    if not np.max(np.abs(y1 - 1.25 * xd * r1) / np.abs(1.25 * xd * r1)) <= 1e-6:
        fails.append("special width-1 y")
    want_dx = dy1 * 1.25 * eps1 * r1 ** 3
    if not np.max(np.abs(dx1 - want_dx) / np.abs(want_dx)) <= 1e-4:
        fails.append("special width-1 dx")
    # scale invariance
    rng = np.random.default_rng(9)
    xs = rng.standard_normal((4, 24)).astype(np.float32)
    gs = rng.uniform(0.5, 1.5, 24).astype(np.float32)
    ya, _ = oracle.fwd(xs, gs, 1e-6, mutation=mutation)
    yb, _ = oracle.fwd((1000.0 * xs).astype(np.float32), gs, 1e-6, mutation=mutation)
    if not row_rel_err(yb, ya) <= 1e-5:
        fails.append("special scale invariance")
    return fails


def check_dgamma_ones(mutation: int = 0):
    fails = []
    rng = np.random.default_rng(13)
    x = rng.standard_normal((37, 20)).astype(np.float32)
    xhat, inv = oracle.fwd(x, None, 1e-6, mutation=mutation)
    dy = np.ones_like(x)
    _, dg = oracle.bwd(x, None, inv, dy, mutation=mutation)
    want = np.sum(xhat.astype(np.float64), axis=0)
    if not vec_rel_err(dg, want) <= 1e-6:
        fails.append("dgamma_ones")
    return fails


def check_permutation(mutation: int = 0):
    fails = []
    rng = np.random.default_rng(17)
    x = rng.standard_normal((29, 12)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, 12).astype(np.float32)
    dy = rng.standard_normal((29, 12)).astype(np.float32)
    perm = rng.permutation(29)
    y, inv = oracle.fwd(x, g, 1e-6, mutation=mutation)
    dx, dg = oracle.bwd(x, g, inv, dy, mutation=mutation)
    yp, invp = oracle.fwd(x[perm], g, 1e-6, mutation=mutation)
    dxp, dgp = oracle.bwd(x[perm], g, invp, dy[perm], mutation=mutation)
    if not (np.array_equal(yp, y[perm]) and np.array_equal(dxp, dx[perm])):
        fails.append("permutation equivariance of y/dx")
    if not vec_rel_err(dgp, dg) <= 1e-6:
        fails.append("permutation invariance of dgamma")
    return fails


def check_accumulate(mutation: int = 0):
    fails = []
    rng = np.random.default_rng(19)
    x = rng.standard_normal((5, 16)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, 16).astype(np.float32)
    dy = rng.standard_normal((5, 16)).astype(np.float32)
    _, inv = oracle.fwd(x, g, 1e-6, mutation=mutation)
    dx0, dg0 = oracle.bwd(x, g, inv, dy, mutation=mutation)
    pre_dx = rng.standard_normal((5, 16)).astype(np.float32)
    pre_dg = rng.standard_normal(16).astype(np.float32)
    dx1, dg1 = oracle.bwd(x, g, inv, dy, mutation=mutation, dx=pre_dx, dgamma=pre_dg,
                          accumulate=True)
    if not np.array_equal(dx1, pre_dx + dx0) or not np.array_equal(dg1, pre_dg + dg0):
        fails.append("accumulate: grad += contribution")
    return fails


def check_linear(mutation: int = 0):
    """matmul + VJP of the c5 layer on small bf16 inputs."""
    fails = []
    rng = np.random.default_rng(23)
    bits = lambda a: oracle.bf16_encode(np.asarray(a, np.float32))  # noqa: E731
    dec = oracle.bf16_decode
    # identity: y == h exactly (products of bf16 values by 1 and 0 are exact)
    h = bits(rng.standard_normal((6, 8)))
    y = oracle.linear_fwd(h, bits(np.eye(8)))
    if not np.array_equal(y, h):
        fails.append("linear identity: y != h")
    # central differences of L = sum(y * dy) in float64 (the bf16 rounding of y
    # is outside the derivative; compare against the exact products)
    hf = dec(bits(rng.standard_normal((5, 7)))).astype(np.float64)
    wf = dec(bits(0.3 * rng.standard_normal((7, 4)))).astype(np.float64)
    dyf = dec(bits(rng.standard_normal((5, 4)))).astype(np.float64)
    dh, dw = oracle.linear_bwd(bits(hf), bits(wf), bits(dyf))

    def loss(hh, ww):
        return float(np.sum(oracle.matmul_f64(hh, ww) * dyf))

    eps = 1e-4
    num_dh = np.zeros_like(hf)
    for i in np.ndindex(hf.shape):
        p, m = hf.copy(), hf.copy()
        p[i] += eps
        m[i] -= eps
        num_dh[i] = (loss(p, wf) - loss(m, wf)) / (2 * eps)
    num_dw = np.zeros_like(wf)
    for i in np.ndindex(wf.shape):
        p, m = wf.copy(), wf.copy()
        p[i] += eps
        m[i] -= eps
        num_dw[i] = (loss(hf, p) - loss(hf, m)) / (2 * eps)
    if not np.max(np.abs(dec(dh) - num_dh)) <= 1e-2 * max(1.0, np.max(np.abs(num_dh))):
        fails.append("linear dh central differences")
    if not np.max(np.abs(dw - num_dw)) <= 1e-6 * max(1.0, np.max(np.abs(num_dw))):
        fails.append("linear dW central differences")
    # the layer composes the RMSNorm VJP with dh
    x = bits(rng.standard_normal((4, 16)))
    g = bits(rng.uniform(0.5, 1.5, 16))
    w = bits(0.2 * rng.standard_normal((16, 8)))
    dy = bits(rng.standard_normal((4, 8)))
    out = oracle.rmsnorm_linear_layer(x, g, w, dy, 1e-5)
    h2, inv2 = oracle.fwd(x, g, 1e-5, mutation=mutation)
    dh2, _ = oracle.linear_bwd(h2, w, dy)
    dx2, dg2 = oracle.bwd(x, g, inv2, dh2, mutation=mutation)
    if not (np.array_equal(out["dx"], dx2) and np.array_equal(out["dgamma"], dg2)):
        fails.append("layer: dx, dgamma != RMSNorm VJP of dh")
    return fails


ALL_CHECKS = (check_golden, check_fd, check_fd_truth, check_invariant, check_special,
              check_dgamma_ones, check_permutation, check_accumulate, check_linear)


def run_all(mutation: int = 0):
    fails = []
    for chk in ALL_CHECKS:
        fails += chk(mutation)
    return fails

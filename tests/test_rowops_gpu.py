"""Parity of the row ops of include/agk_rowops.h with the pinned oracle (oracle/rowops.py).

Every op runs on the GPU through the C ABI on a full tensor; rows are
independent, so the oracle checks all rows of small cases and a fixed sample
of rows (first, last, random) of large ones.  Bars (tests/tolerances.py):
fp32 storage 1e-5, bf16 storage 1e-2, per row, relative to the row's scale:
  - outputs that are plain values (y of LayerNorm / softmax, log-sum-exp,
    the log-sum-exp VJP): max|d| / max|ref| per row;
  - outputs that are a difference of terms (LayerNorm dx, softmax dz, the
    RMSNorm and log-sum-exp JVPs): max|d| over the sum of the terms' per-row
    magnitudes, the only bound fp32 can meet where the terms cancel;
  - per-row statistics (mean, rstd): 1e-5 (fp32 arithmetic either way).
Also covered: every resident launch shape (at its narrowest and widest
width, below and above the large-batch threshold), widths that take the
looped kernels (16-byte and element-wise), misaligned pointers, masked (-inf) entries, accumulation,
run-to-run determinism and full-size configurations through properties.
"""
from __future__ import annotations

import numpy as np
import pytest

import cgadimpl_amd as agk
from gpu_util import as_f32, device_inputs, to_host
from oracle import rowops as ro
from tolerances import TOL_BF16, TOL_F32

pytestmark = pytest.mark.gpu

OPS = ("rmsnorm_jvp", "layernorm", "softmax", "logsumexp")
# ... including vocabulary widths past the resident shapes (128256 = Llama 3's
# vocabulary): aligned rows take the 16-byte looped kernel; rows that are not
# whole 16-byte slots from 8192 columns (8193, 131076 bf16, 50257 = GPT-2's
# vocabulary, where every row starts at another offset) its head/body/tail
# form; narrower ones the element-wise kernel.
SHAPES = [(5, 1), (3, 3), (17, 13), (9, 100), (33, 127), (65, 129), (8, 1000), (37, 4096),
          (4, 4099), (2, 40000), (300, 64), (1000, 128), (512, 512), (64, 5120), (3, 65536),
          (4, 128256), (2, 131076), (1, 262144), (9, 50257), (5, 8193)]
EPS = 1e-5


def _tol(bf16):
    return TOL_BF16 if bf16 else TOL_F32


def _sample_rows(R, seed, n=254):
    if R <= n + 2:
        return np.arange(R)
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, R - 1], rng.integers(0, R, n)]))


def _host_rows(t, rows):
    import torch
    if t is None:
        return None
    if t.dim() == 1:  # column vector: not per row
        return to_host(t)
    idx = torch.from_numpy(rows).to(t.device)
    return to_host(t[idx].contiguous())


def _f64(a):
    return as_f32(a).astype(np.float64)


def _rowmax(a):
    return np.max(np.abs(a), axis=-1)


def _scaled_err(got, ref, scale):
    d = _rowmax(_f64(got) - _f64(ref))
    if not np.all(np.isfinite(as_f32(got))):
        return float("inf")
    return float(np.max(np.where(scale > 0, d / np.where(scale > 0, scale, 1.0), d)))


def _row_rel(got, ref):
    return _scaled_err(got, ref, _rowmax(_f64(ref)))


# ---- per-op runners: GPU on full tensors, oracle on sampled rows ----------------------

def check_rmsnorm_jvp(x, g, t, label):
    """ty for the scaled layer (with and without a gamma tangent) and the bare node."""
    import torch
    bf16 = x.dtype == torch.bfloat16
    tg = torch.flip(g, [0]).contiguous() - 1.0
    _, inv = agk.rmsnorm_fwd(x, g, EPS)
    ty = agk.rmsnorm_jvp(x, g, inv, t, tg)
    ty_nog = agk.rmsnorm_jvp(x, g, inv, t, None)
    _, inv0 = agk.rmsnorm_fwd(x, None, EPS)
    ty0 = agk.rmsnorm_jvp(x, None, inv0, t, None)
    torch.cuda.synchronize()
    rows = _sample_rows(x.shape[0], x.shape[1])
    xs, ts = _host_rows(x, rows), _host_rows(t, rows)
    gs, tgs = to_host(g), to_host(tg)
    xf, tf, gf, tgf = _f64(xs), _f64(ts), _f64(gs), _f64(tgs)
    D = xf.shape[-1]
    r = 1.0 / np.sqrt(np.mean(xf * xf, -1) + EPS)
    dot = np.sum(tf * xf, -1)
    t1 = r * _rowmax(gf * tf)
    t2 = r ** 3 * _rowmax(gf * xf) * np.abs(dot) / D
    t3 = r * _rowmax(tgf * xf)
    if bf16:
        ref = ro.rmsnorm_jvp_bf16(xs, gs, ts, tgs, EPS)
        ref_nog = ro.rmsnorm_jvp_bf16(xs, gs, ts, None, EPS)
        ref0 = ro.rmsnorm_jvp_bf16(xs, None, ts, None, EPS)
    else:
        ref = ro.rmsnorm_jvp(xs, gs, ts, tgs, EPS)
        ref_nog = ro.rmsnorm_jvp(xs, gs, ts, None, EPS)
        ref0 = ro.rmsnorm_jvp(xs, None, ts, None, EPS)
    e = {
        "ty": _scaled_err(_host_rows(ty, rows), ref, t1 + t2 + t3),
        "ty_no_tgamma": _scaled_err(_host_rows(ty_nog, rows), ref_nog, t1 + t2),
        "ty_node": _scaled_err(_host_rows(ty0, rows), ref0,
                               r * _rowmax(tf) + r ** 3 * _rowmax(xf) * np.abs(dot) / D),
    }
    return e


def check_layernorm(x, dy, label, eps=EPS):
    import torch
    bf16 = x.dtype == torch.bfloat16
    y, mean, rstd = agk.layernorm_fwd(x, eps)
    dx = agk.layernorm_bwd(x, mean, rstd, dy)
    torch.cuda.synchronize()
    rows = _sample_rows(x.shape[0], x.shape[1] + 1)
    xs, dys = _host_rows(x, rows), _host_rows(dy, rows)
    if bf16:
        ry, rmean, rvar = ro.layernorm_fwd_bf16(xs, eps)
        rdx = ro.layernorm_bwd_bf16(xs, rmean, rvar, dys, eps)
    else:
        ry, rmean, rvar = ro.layernorm_fwd(xs, eps)
        rdx = ro.layernorm_bwd(xs, rmean, rvar, dys, eps)
    xf, gf = _f64(xs), _f64(dys)
    rm, rv = rmean.astype(np.float64)[:, 0], rvar.astype(np.float64)[:, 0]
    rs = 1.0 / np.sqrt(rv + eps)
    xhat = (xf - rm[:, None]) * rs[:, None]
    scale = rs * (_rowmax(gf) + np.abs(gf.mean(-1)) + _rowmax(xhat) * np.abs((gf * xhat).mean(-1)))
    gm = _host_rows(mean, rows).reshape(-1).astype(np.float64)
    gr = _host_rows(rstd, rows).reshape(-1).astype(np.float64)
    e = {
        "y": _row_rel(_host_rows(y, rows), ry),
        "mean": float(np.max(np.abs(gm - rm) / np.maximum(_rowmax(xf), 1e-30))),
        "rstd": float(np.max(np.abs(gr - rs) / rs)),
        "dx": _scaled_err(_host_rows(dx, rows), rdx, scale),
    }
    return e


def check_softmax(z, dy, label):
    import torch
    bf16 = z.dtype == torch.bfloat16
    y = agk.softmax_fwd(z)
    dz = agk.softmax_bwd(y, dy)
    torch.cuda.synchronize()
    rows = _sample_rows(z.shape[0], z.shape[1] + 2)
    zs, dys, ys = _host_rows(z, rows), _host_rows(dy, rows), _host_rows(y, rows)
    if bf16:
        ry = ro.softmax_fwd_bf16(zs)
        rdz = ro.softmax_bwd_bf16(ys, dys)   # the backward from the GPU's own y
    else:
        ry = ro.softmax_fwd(zs)
        rdz = ro.softmax_bwd(ys, dys)
    yf, gf = _f64(ys), _f64(dys)
    scale = _rowmax(yf) * (_rowmax(gf) + np.abs(np.sum(yf * gf, -1)))
    return {"y": _row_rel(ys, ry), "dz": _scaled_err(_host_rows(dz, rows), rdz, scale)}


def check_logsumexp(z, t, label):
    import torch
    bf16 = z.dtype == torch.bfloat16
    R = z.shape[0]
    dy = t[:, :1].contiguous() if t.shape[1] else torch.ones(R, 1, dtype=z.dtype,
                                                             device=z.device)
    y = agk.logsumexp_fwd(z)
    dz = agk.logsumexp_bwd(z, dy)
    ty = agk.logsumexp_jvp(z, t)
    # the forward that keeps its fp32 value, and the one-pass backward from it
    yk, lse = agk.logsumexp_fwd_keep(z)
    dzv = agk.logsumexp_bwd_from_value(z, lse, dy)
    torch.cuda.synchronize()
    assert torch.equal(yk, y), f"{label}: logsumexp_fwd_keep's y differs from logsumexp_fwd's"
    rows = _sample_rows(R, z.shape[1] + 3)
    zs, ts, dys = _host_rows(z, rows), _host_rows(t, rows), _host_rows(dy, rows)
    if bf16:
        ry, rdz, rty = (ro.logsumexp_fwd_bf16(zs), ro.logsumexp_bwd_bf16(zs, dys),
                        ro.logsumexp_jvp_bf16(zs, ts))
    else:
        ry, rdz, rty = ro.logsumexp_fwd(zs), ro.logsumexp_bwd(zs, dys), ro.logsumexp_jvp(zs, ts)
    rl32 = ro.logsumexp_fwd(as_f32(zs))  # the fp32 value the storage-type y rounds
    zf = _f64(zs)
    sm = np.exp(zf - zf.max(-1, keepdims=True))
    sm /= sm.sum(-1, keepdims=True)
    jscale = np.sum(np.abs(sm * _f64(ts)), -1)
    lscale = np.maximum(np.abs(_f64(rl32))[:, 0], 1.0)
    return {
        "y": _scaled_err(_host_rows(y, rows), ry, np.maximum(np.abs(_f64(ry))[:, 0], 1.0)),
        "dz": _row_rel(_host_rows(dz, rows), rdz),
        "ty": _scaled_err(_host_rows(ty, rows), rty, jscale),
        # fp32 whatever the storage: held to the fp32 bar
        "lse": _scaled_err(_host_rows(lse, rows), rl32, lscale) * (_tol(bf16) / TOL_F32),
        "dz from lse": _row_rel(_host_rows(dzv, rows), rdz),
    }


def run_op(op, x, g, dy, label):
    if op == "rmsnorm_jvp":
        return check_rmsnorm_jvp(x, g, dy, label)
    if op == "layernorm":
        return check_layernorm(x, dy, label)
    if op == "softmax":
        return check_softmax(x * 4.0, dy, label)
    return check_logsumexp(x * 4.0, dy, label)


def assert_ok(e, tol, label):
    print(f"[{label}] " + " ".join(f"{k}={v:.2e}" for k, v in e.items()), flush=True)
    for k, v in e.items():
        lim = TOL_F32 if k in ("mean", "rstd") else tol
        assert v <= lim, (label, k, v, lim)


# ---- cases ------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("rows,cols", SHAPES, ids=lambda v: str(v))
@pytest.mark.parametrize("op", OPS)
def test_op_matches_oracle(cuda, op, rows, cols, dtype):
    dt = agk.AGK_F32 if dtype == "f32" else agk.AGK_BF16
    p = agk.launch_plan(rows, cols, dt, False)
    label = f"{op} {dtype} {rows}x{cols} plan{(p['tpr'], p['nv'], p['g'])}"
    print(label, flush=True)
    x, g, dy = device_inputs((rows, cols), dtype, rows * 1009 + cols, cuda)
    assert_ok(run_op(op, x, g, dy, label), _tol(dtype == "bf16"), label)


def _plan_cases():
    from plans import reachable_plans
    seen, cases = set(), []
    for (dt, direction, _tpr, _nv, _g), reps in sorted(reachable_plans().items()):
        if direction != "fwd":
            continue
        for rows, cols in reps:
            key = ("f32" if dt == agk.AGK_F32 else "bf16", rows, cols)
            if key not in seen:
                seen.add(key)
                cases.append(key)
    return cases


@pytest.mark.parametrize("dtype,rows,cols", _plan_cases(), ids=lambda v: str(v))
def test_every_launch_shape(cuda, dtype, rows, cols):
    """All four ops at every resident shape the row plan can pick."""
    dt = agk.AGK_F32 if dtype == "f32" else agk.AGK_BF16
    p = agk.launch_plan(rows, cols, dt, False)
    x, g, dy = device_inputs((rows, cols), dtype, rows * 31 + cols, cuda)
    for op in OPS:
        label = f"{op} {dtype} {rows}x{cols} plan{(p['tpr'], p['nv'], p['g'])}"
        print(label, flush=True)
        assert_ok(run_op(op, x, g, dy, label), _tol(dtype == "bf16"), label)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("op", OPS)
def test_misaligned_pointers_take_the_looped_kernel(cuda, op, dtype):
    import torch
    rows, cols = 24, 256
    x, g, dy = device_inputs((rows, cols), dtype, 77, cuda)

    def shifted(t):  # same values, 1 element past a 16-byte boundary
        buf = torch.empty(t.numel() + 8, dtype=t.dtype, device=t.device)
        v = buf[1:1 + t.numel()].view(t.shape)
        v.copy_(t)
        return v

    label = f"{op} {dtype} misaligned"
    print(label, flush=True)
    e_al = run_op(op, x, g, dy, label + " (aligned)")
    e_mis = run_op(op, shifted(x), shifted(g), shifted(dy), label)
    assert_ok(e_mis, _tol(dtype == "bf16"), label)
    assert_ok(e_al, _tol(dtype == "bf16"), label + " (aligned)")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("cols", [40000, 50257])
def test_same_offset_tensors_take_the_16_byte_kernel(cuda, dtype, cols):
    """Every tensor one element off a 16-byte boundary (inputs and outputs at
    the same offset), at a width past the resident shapes: softmax and
    log-sum-exp forward and backward through the head/body/tail form of the
    16-byte looped kernel, against the oracle with check_softmax's and
    check_logsumexp's bars."""
    import torch
    rows = 5
    x, _, dy = device_inputs((rows, cols), dtype, 79 + cols, cuda)

    def shifted(t):  # same values, one element past a 16-byte boundary
        buf = torch.empty(t.numel() + 8, dtype=t.dtype, device=t.device)
        v = buf[1:1 + t.numel()].view(t.shape)
        v.copy_(t)
        return v

    z, d = shifted(x * 4.0), shifted(dy)
    y, dz, dlz = shifted(torch.zeros_like(x)), shifted(torch.zeros_like(x)), \
        shifted(torch.zeros_like(x))
    assert z.data_ptr() % 16 != 0 and (y.data_ptr() - z.data_ptr()) % 16 == 0
    agk.softmax_fwd(z, y=y)
    agk.softmax_bwd(y, d, dz=dz)
    dl = dy[:, :1].contiguous()
    lse = agk.logsumexp_fwd(z)
    agk.logsumexp_bwd(z, dl, dz=dlz)
    _, l32 = agk.logsumexp_fwd_keep(z)
    dlv = shifted(torch.zeros_like(x))
    agk.logsumexp_bwd_from_value(z, l32, dl, dz=dlv)  # head/body/tail form
    torch.cuda.synchronize()
    zs, ds, ys, dls = to_host(z), to_host(d), to_host(y), to_host(dl)
    bf16 = dtype == "bf16"
    if bf16:
        ry, rdz = ro.softmax_fwd_bf16(zs), ro.softmax_bwd_bf16(ys, ds)
        rl, rdl = ro.logsumexp_fwd_bf16(zs), ro.logsumexp_bwd_bf16(zs, dls)
    else:
        ry, rdz = ro.softmax_fwd(zs), ro.softmax_bwd(ys, ds)
        rl, rdl = ro.logsumexp_fwd(zs), ro.logsumexp_bwd(zs, dls)
    yf, gf = _f64(ys), _f64(ds)
    scale = _rowmax(yf) * (_rowmax(gf) + np.abs(np.sum(yf * gf, -1)))
    e = {"softmax y": _row_rel(ys, ry), "softmax dz": _scaled_err(to_host(dz), rdz, scale),
         "lse y": _scaled_err(to_host(lse), rl, np.maximum(np.abs(_f64(rl))[:, 0], 1.0)),
         "lse dz": _row_rel(to_host(dlz), rdl),
         "lse dz from value": _row_rel(to_host(dlv), rdl)}
    assert_ok(e, _tol(bf16), f"same-offset {dtype} {rows}x{cols}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(40, 384), (3, 131072)], ids=str)
def test_backward_accumulates(cuda, dtype, shape):
    import torch
    x, g, dy = device_inputs(shape, dtype, 5, cuda)
    pre = torch.randn(x.shape, device=cuda).to(x.dtype)
    y, mean, rstd = agk.layernorm_fwd(x)
    outs = {
        "layernorm": (agk.layernorm_bwd(x, mean, rstd, dy),
                      agk.layernorm_bwd(x, mean, rstd, dy, dx=pre.clone(), accumulate=True)),
    }
    s = agk.softmax_fwd(x)
    outs["softmax"] = (agk.softmax_bwd(s, dy),
                       agk.softmax_bwd(s, dy, dz=pre.clone(), accumulate=True))
    dr = dy[:, :1].contiguous()
    outs["logsumexp"] = (agk.logsumexp_bwd(x, dr),
                         agk.logsumexp_bwd(x, dr, dz=pre.clone(), accumulate=True))
    _, l32 = agk.logsumexp_fwd_keep(x)
    outs["logsumexp from value"] = (
        agk.logsumexp_bwd_from_value(x, l32, dr),
        agk.logsumexp_bwd_from_value(x, l32, dr, dz=pre.clone(), accumulate=True))
    torch.cuda.synchronize()
    tol = 2 * _tol(dtype == "bf16")
    for name, (fresh, acc) in outs.items():
        want = pre.double() + fresh.double()
        err = float(((acc.double() - want).abs().max() / want.abs().max()).item())
        print(f"[accumulate {name} {dtype}] {err:.2e}", flush=True)
        assert err <= tol, (name, err)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("cols", [96, 131072])
def test_masked_entries(cuda, dtype, cols):
    """-inf entries (masked logits) get probability 0 and drop out of the log-sum-exp."""
    import torch
    z = torch.randn(16, cols, device=cuda) * 3
    z[:, ::3] = float("-inf")
    z = z.to(torch.bfloat16 if dtype == "bf16" else torch.float32).contiguous()
    y = agk.softmax_fwd(z)
    lse = agk.logsumexp_fwd(z)
    torch.cuda.synchronize()
    assert torch.all(y[:, ::3] == 0)
    keep = z.float()[:, [j for j in range(cols) if j % 3]]
    want = torch.logsumexp(keep.double(), -1, keepdim=True)
    assert float((lse.double() - want).abs().max()) <= _tol(dtype == "bf16") * float(
        want.abs().max())
    assert float((y.double().sum(-1) - 1).abs().max()) <= 2 * _tol(dtype == "bf16")


# a resident width, a bf16 width of the 16-slot resident shape (32769-65536),
# GPT-2's unaligned vocabulary (head/body/tail looped kernel, online max and
# sum) and an aligned looped width
@pytest.mark.parametrize("dtype,cols", [("f32", 96), ("bf16", 40000), ("bf16", 50257),
                                        ("f32", 50257), ("bf16", 262144)])
def test_fully_masked_rows_are_nan(cuda, dtype, cols):
    """A row that is -inf throughout: the reference's two-pass rule
    (reduction.cpp:42-66) computes exp(-inf - -inf) = NaN, and so does the
    oracle; every kernel path gives NaN for softmax and log-sum-exp there, and
    the other rows stay finite and match the oracle."""
    import warnings
    import torch
    z = torch.randn(4, cols, device=cuda) * 3
    z[1] = float("-inf")
    z = z.to(torch.bfloat16 if dtype == "bf16" else torch.float32).contiguous()
    y = agk.softmax_fwd(z)
    lse = agk.logsumexp_fwd(z)
    torch.cuda.synchronize()
    zh = as_f32(to_host(z))
    with warnings.catch_warnings(), np.errstate(invalid="ignore"):
        warnings.simplefilter("ignore", RuntimeWarning)
        ry = ro.softmax_fwd(zh)
        rl = ro.logsumexp_fwd(zh)
    assert np.all(np.isnan(ry[1])) and np.isnan(rl[1]).all()  # the oracle's own rule
    yh, lh = as_f32(to_host(y)), as_f32(to_host(lse)).reshape(4, 1)
    assert np.all(np.isnan(yh[1])), "softmax of a fully masked row"
    assert np.isnan(lh[1]).all(), "log-sum-exp of a fully masked row"
    keep = [0, 2, 3]
    assert np.all(np.isfinite(yh[keep])) and np.all(np.isfinite(lh[keep]))
    tol = _tol(dtype == "bf16")
    assert _row_rel(yh[keep], ry[keep]) <= tol
    assert np.abs(lh[keep] - rl[keep]).max() <= tol * np.abs(rl[keep]).max()


@pytest.mark.parametrize("shape", [(4099, 1000), (7, 131072)], ids=str)
def test_results_are_deterministic(cuda, shape):
    import torch
    x, g, dy = device_inputs(shape, "f32", 3, cuda)
    first = None
    for _ in range(3):
        y, mean, rstd = agk.layernorm_fwd(x)
        l32 = agk.logsumexp_fwd_keep(x)[1]
        outs = [y, mean, rstd, agk.layernorm_bwd(x, mean, rstd, dy), agk.softmax_fwd(x),
                agk.logsumexp_fwd(x), agk.logsumexp_jvp(x, dy), l32,
                agk.logsumexp_bwd_from_value(x, l32, dy[:, :1].contiguous())]
        torch.cuda.synchronize()
        if first is None:
            first = [o.clone() for o in outs]
        else:
            for a, b in zip(first, outs):
                assert torch.equal(a, b)


# ---- full-size configurations -------------------------------------------------------

@pytest.mark.slow
@pytest.mark.parametrize("name", ["c2", "c3"])
def test_full_size(cuda, name):
    """[32,2048,4096] fp32 and [16,4096,8192] bf16: sampled rows against the
    oracle, plus properties over every row in fp64 on the device."""
    import torch
    from cgadimpl_amd import configs
    cfg = configs.CONFIGS[name]
    R, D = cfg.rows, cfg.cols
    bf16 = cfg.dtype == "bf16"
    x, g, dy = device_inputs((R, D), cfg.dtype, cfg.seed, cuda)
    tol = _tol(bf16)
    for op in OPS:
        label = f"{op} full-size {name}"
        print(label, flush=True)
        assert_ok(run_op(op, x, g, dy, label), tol, label)
    # softmax rows sum to 1, LayerNorm rows have mean 0 and variance var/(var+eps)
    y = agk.softmax_fwd(x)
    s = y.double().sum(-1)
    assert float((s - 1).abs().max()) <= (2.0 ** -7 if bf16 else 1e-5)
    ln, mean, rstd = agk.layernorm_fwd(x)
    lnd = ln.double()
    assert float(lnd.mean(-1).abs().max()) <= (1e-2 if bf16 else 1e-5)
    del y, s, ln, lnd
    # adjoint identity between the RMSNorm JVP and the (separately pinned) VJP
    tg = torch.flip(g, [0]).contiguous() - 1.0
    _, inv = agk.rmsnorm_fwd(x, g, EPS)
    ty = agk.rmsnorm_jvp(x, g, inv, dy, tg)
    w = torch.randn(x.shape, device=cuda).to(x.dtype)
    dx, dgam = agk.rmsnorm_bwd(x, g, inv, w)
    torch.cuda.synchronize()
    lhs = float((w.double() * ty.double()).sum())
    rhs = float((dx.double() * dy.double()).sum() + (dgam.double() * tg.double()).sum())
    rel = abs(lhs - rhs) / max(abs(rhs), float((w.double() * ty.double()).abs().sum()) * 1e-3)
    print(f"[{name}] adjoint identity <w, J t> vs <J^T w, t>: {rel:.2e}", flush=True)
    assert rel <= (5e-2 if bf16 else 1e-4)


# ---- rows over several workgroups: the *_ws entry points' team kernel -------------------

# Vocabulary widths and one row per team: aligned rows of many parts (Llama 3's
# 128256, Qwen's 151936, 2^19), rows that start at another offset in every row
# (GPT-2's 50257), more rows than teams (each team then runs several rows, odd
# and even counts), one row.
TEAM_SHAPES = [("bf16", 700, 128256), ("f32", 65, 128256), ("bf16", 1, 151936),
               ("bf16", 33, 50257), ("f32", 9, 50257), ("bf16", 3, 1 << 19),
               ("f32", 130, 40000), ("f32", 2, 8193)]


def _team_parts(dtype, rows, cols, aligned):
    """Workgroups per row of the team launch (the most of the three ops: the
    softmax backward takes rows off a 16-byte boundary from fewer parts)."""
    return max(agk.rowops_team_plan(op, rows, cols, 0 if dtype == "f32" else 1, aligned)["parts"]
               for op in agk.ROWOPS_TEAM_OPS)


def _softmax_lse_outputs(z, dy, dl, ws):
    y = agk.softmax_fwd(z, workspace=ws)
    dz = agk.softmax_bwd(y, dy, workspace=ws)
    dlz = agk.logsumexp_bwd(z, dl, workspace=ws)
    return y, dz, dlz


@pytest.mark.parametrize("dtype,rows,cols", TEAM_SHAPES, ids=str)
def test_team_rows_match_oracle_and_recompute(cuda, dtype, rows, cols):
    """Softmax forward and backward and the log-sum-exp backward on the team
    kernel (a row over several workgroups that exchange their partial sums):
    against the oracle with check_softmax's and check_logsumexp's bars, against
    the workspace-free kernels within the same bars (the row sums are added in
    another order), and with every wait cut to its first look (wait limit 0:
    the workgroups recompute the partial sums they do not find yet)
    bit-identical to the default -- a recomputed partial sum is the published
    one."""
    import torch
    aligned = cols % (4 if dtype == "f32" else 8) == 0
    parts = _team_parts(dtype, rows, cols, aligned)
    print(f"team rowops {dtype} {rows}x{cols} parts {parts}", flush=True)
    assert parts >= 2, "the shape should take the team kernel"
    x, _, dy = device_inputs((rows, cols), dtype, rows + cols, cuda)
    z = x * 4.0
    dl = dy[:, :1].contiguous()
    team = _softmax_lse_outputs(z, dy, dl, None)
    plain = _softmax_lse_outputs(z, dy, dl, False)
    prev = agk.set_exchange_wait_limit(0)
    try:
        rec = _softmax_lse_outputs(z, dy, dl, None)
    finally:
        agk.set_exchange_wait_limit(prev)
    torch.cuda.synchronize()
    for a, b in zip(team, rec):
        assert torch.equal(a, b)
    y, dz, dlz = team
    bf16 = dtype == "bf16"
    srows = _sample_rows(rows, cols)
    zs, dys, ys, dls = (_host_rows(z, srows), _host_rows(dy, srows), _host_rows(y, srows),
                        _host_rows(dl, srows))
    if bf16:
        ry, rdz, rdl = (ro.softmax_fwd_bf16(zs), ro.softmax_bwd_bf16(ys, dys),
                        ro.logsumexp_bwd_bf16(zs, dls))
    else:
        ry, rdz, rdl = ro.softmax_fwd(zs), ro.softmax_bwd(ys, dys), ro.logsumexp_bwd(zs, dls)
    yf, gf = _f64(ys), _f64(dys)
    scale = _rowmax(yf) * (_rowmax(gf) + np.abs(np.sum(yf * gf, -1)))
    py, pdz, pdl = (_host_rows(t, srows) for t in plain)
    e = {"y": _row_rel(ys, ry), "dz": _scaled_err(_host_rows(dz, srows), rdz, scale),
         "lse dz": _row_rel(_host_rows(dlz, srows), rdl),
         "y vs workspace-free": _row_rel(ys, py),
         "dz vs workspace-free": _scaled_err(_host_rows(dz, srows), pdz, scale),
         "lse dz vs workspace-free": _row_rel(_host_rows(dlz, srows), pdl)}
    assert_ok(e, _tol(bf16), f"team {dtype} {rows}x{cols}")


def test_team_rowops_on_two_streams_at_once(cuda):
    """The row ops' team kernels of two calls running at once on two streams
    (default priority; together more workgroups than the GPU holds at once):
    every output bit-identical to the same calls made one after the other."""
    import torch
    rows, cols = 2048, 128256
    x, _, dy = device_inputs((rows, cols), "bf16", 17, cuda)
    z = x * 4.0
    dl = dy[:, :1].contiguous()
    ref = (agk.softmax_fwd(z), agk.logsumexp_bwd(z, dl))
    ref_b = agk.softmax_bwd(ref[0], dy)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    ws = [torch.empty(agk.rowops_workspace_bytes(rows, cols), dtype=torch.uint8, device=cuda)
          for _ in range(3)]
    for rep in range(3):
        with torch.cuda.stream(s1):
            y = agk.softmax_fwd(z, workspace=ws[0], stream=s1)
            dzb = agk.softmax_bwd(ref[0], dy, workspace=ws[2], stream=s1)
        with torch.cuda.stream(s2):
            dz = agk.logsumexp_bwd(z, dl, workspace=ws[1], stream=s2)
        torch.cuda.synchronize()
        print(f"row ops on two streams, round {rep}", flush=True)
        assert torch.equal(y, ref[0]) and torch.equal(dz, ref[1]) and torch.equal(dzb, ref_b), rep


@pytest.mark.parametrize("dtype,cols", [("bf16", 131072), ("f32", 131072), ("f32", 100000)],
                         ids=str)
def test_team_masked_ranges(cuda, dtype, cols):
    """Team rows where whole parts are -inf (masked spans wider than a part's
    range, 16384 bf16 or 8192 fp32 elements): a part whose maximum is -inf
    contributes nothing, its outputs are 0, and the other parts' outputs match
    the oracle; a row that is -inf throughout gives NaN, as on the other paths.
    Softmax forward and the log-sum-exp backward (the kernels that keep each
    part's exponentials), with the workspace-free kernels within the bars."""
    import warnings
    import torch
    rows = 6
    bf16 = dtype == "bf16"
    aligned = cols % (8 if bf16 else 4) == 0
    assert _team_parts(dtype, rows, cols, aligned) >= 2
    z = torch.randn(rows, cols, device=cuda) * 3
    z[0, :40000] = float("-inf")           # the first parts, and part of the next
    z[1, cols - 50000:] = float("-inf")    # the last parts
    z[2, 20000:90000] = float("-inf")      # parts in the middle
    z[3] = float("-inf")                   # the whole row
    z[4, :] = float("-inf")
    z[4, 70000] = 1.5                      # one finite element
    z = z.to(torch.bfloat16 if bf16 else torch.float32).contiguous()
    dl = torch.randn(rows, 1, device=cuda).to(z.dtype)
    y = agk.softmax_fwd(z)
    dz = agk.logsumexp_bwd(z, dl)
    y0 = agk.softmax_fwd(z, workspace=False)
    dz0 = agk.logsumexp_bwd(z, dl, workspace=False)
    torch.cuda.synchronize()
    zh, dlh = to_host(z), to_host(dl)
    with warnings.catch_warnings(), np.errstate(invalid="ignore"):
        warnings.simplefilter("ignore", RuntimeWarning)
        if bf16:
            ry, rdz = ro.softmax_fwd_bf16(zh), ro.logsumexp_bwd_bf16(zh, dlh)
        else:
            ry, rdz = ro.softmax_fwd(zh), ro.logsumexp_bwd(zh, dlh)
    yh, dzh = as_f32(to_host(y)), as_f32(to_host(dz))
    masked = np.isneginf(as_f32(zh))
    live = [0, 1, 2, 4, 5]
    assert np.all(np.isnan(yh[3])) and np.all(np.isnan(dzh[3])), "a fully masked row is NaN"
    for r in live:
        assert np.all(yh[r][masked[r]] == 0) and np.all(dzh[r][masked[r]] == 0), r
    assert yh[4, 70000] == 1.0
    tol = _tol(bf16)
    e = {"y": _row_rel(yh[live], ry[live]), "lse dz": _row_rel(dzh[live], rdz[live]),
         "y vs workspace-free": _row_rel(yh[live], as_f32(to_host(y0))[live]),
         "lse dz vs workspace-free": _row_rel(dzh[live], as_f32(to_host(dz0))[live])}
    assert_ok(e, tol, f"team masked ranges {dtype} {rows}x{cols}")


@pytest.mark.parametrize("dtype,rows,cols", [("bf16", 50, 4096), ("f32", 300, 2048),
                                             ("bf16", 20, 20000), ("f32", 17, 10001),
                                             ("bf16", 5, 65536)], ids=str)
def test_team_kernel_on_narrow_rows(cuda, dtype, rows, cols):
    """Mode 2 puts rows the default keeps on one workgroup (one part, two or
    three parts, a last part holding the tail) on the team kernel: the same
    bars against the oracle, and the recompute path bit-identical."""
    import torch
    bf16 = dtype == "bf16"
    prev = agk.set_rowops_team(2)
    try:
        aligned = cols % (8 if bf16 else 4) == 0
        assert _team_parts(dtype, rows, cols, aligned) >= 1
        x, _, dy = device_inputs((rows, cols), dtype, 3 * rows + cols, cuda)
        z = x * 4.0
        dl = dy[:, :1].contiguous()
        ws = torch.empty(rows * 64 * 16, dtype=torch.uint8, device=cuda)
        y, dz, dlz = _softmax_lse_outputs(z, dy, dl, ws)
        pw = agk.set_exchange_wait_limit(0)
        try:
            rec = _softmax_lse_outputs(z, dy, dl, ws)
        finally:
            agk.set_exchange_wait_limit(pw)
    finally:
        agk.set_rowops_team(prev)
    torch.cuda.synchronize()
    for a, b in zip((y, dz, dlz), rec):
        assert torch.equal(a, b)
    zs, dys, ys, dls = to_host(z), to_host(dy), to_host(y), to_host(dl)
    if bf16:
        ry, rdz, rdl = (ro.softmax_fwd_bf16(zs), ro.softmax_bwd_bf16(ys, dys),
                        ro.logsumexp_bwd_bf16(zs, dls))
    else:
        ry, rdz, rdl = ro.softmax_fwd(zs), ro.softmax_bwd(ys, dys), ro.logsumexp_bwd(zs, dls)
    yf, gf = _f64(ys), _f64(dys)
    scale = _rowmax(yf) * (_rowmax(gf) + np.abs(np.sum(yf * gf, -1)))
    e = {"y": _row_rel(ys, ry), "dz": _scaled_err(to_host(dz), rdz, scale),
         "lse dz": _row_rel(to_host(dlz), rdl)}
    assert_ok(e, _tol(bf16), f"team mode 2 {dtype} {rows}x{cols}")


@pytest.mark.parametrize("dtype,cols", [("bf16", 131072), ("f32", 50257)], ids=str)
def test_team_accumulates_and_is_deterministic(cuda, dtype, cols):
    """The team kernel's backward outputs add into dz as the other kernels do
    (fp32: pre + fresh within one rounding; bf16 within two), and three calls
    give the same bits."""
    import torch
    rows = 37
    x, _, dy = device_inputs((rows, cols), dtype, 11, cuda)
    assert _team_parts(dtype, rows, cols, cols % 8 == 0) >= 2
    pre = torch.randn(x.shape, device=cuda).to(x.dtype)
    s = agk.softmax_fwd(x)
    dl = dy[:, :1].contiguous()
    outs = {"softmax": (agk.softmax_bwd(s, dy), agk.softmax_bwd(s, dy, dz=pre.clone(),
                                                                accumulate=True)),
            "logsumexp": (agk.logsumexp_bwd(x, dl),
                          agk.logsumexp_bwd(x, dl, dz=pre.clone(), accumulate=True))}
    first = [agk.softmax_fwd(x), agk.softmax_bwd(s, dy), agk.logsumexp_bwd(x, dl)]
    for _ in range(2):
        again = [agk.softmax_fwd(x), agk.softmax_bwd(s, dy), agk.logsumexp_bwd(x, dl)]
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(first, again))
    tol = 2 * _tol(dtype == "bf16")
    for name, (fresh, acc) in outs.items():
        want = pre.double() + fresh.double()
        err = float(((acc.double() - want).abs().max() / want.abs().max()).item())
        print(f"[team accumulate {name} {dtype}] {err:.2e}", flush=True)
        assert err <= tol, (name, err)

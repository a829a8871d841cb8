"""Parity of the HIP path (through the C ABI) with the pinned CPU oracle.

Bars: fp32 storage per-row max|d| / max|ref| <= 1e-5 for y and dx, the same
norm-wise bound for dgamma; bf16 storage 1e-2; inv_rms 1e-5 relative; dgamma
bit-identical across repeated runs.  Sizes: every configuration at a size the
oracle finishes in seconds (full size where it does), and the full-size
configurations through size-independent properties (oracle on sampled rows,
fp64 dgamma, the sum_j x_j dx_j identity, determinism).
"""
import os

import numpy as np
import pytest

import cgadimpl_amd as agk
import oracle
import pins
from cgadimpl_amd import configs
from gpu_util import as_f32, gpu_layer, to_dev, to_host
from tolerances import TOL_BF16, TOL_F32, dx_rel_err, row_rel_err, vec_rel_err

pytestmark = pytest.mark.gpu

NTHREADS = max(1, min(16, len(os.sched_getaffinity(0))))


@pytest.fixture(scope="module", autouse=True)
def _oracle_threads():
    oracle.set_threads(NTHREADS)
    yield
    oracle.set_threads(1)


def _tol(x):
    return TOL_BF16 if x.dtype == np.uint16 else TOL_F32


def _compare(x, gamma, dy, eps, got, label, check_dg=True):
    y, inv, dx, dg = got
    ry, rinv = oracle.fwd(x, gamma, eps)
    rdx, rdg = oracle.bwd(x, gamma, rinv, dy)
    tol = _tol(x)
    e = {
        "y": row_rel_err(as_f32(y), as_f32(ry)),
        "inv_rms": vec_rel_err(inv, rinv),
        "dx": dx_rel_err(as_f32(dx), as_f32(rdx), as_f32(x), as_f32(gamma), as_f32(dy), eps),
    }
    if check_dg:
        e["dgamma"] = vec_rel_err(dg, rdg)
    print(f"[{label}] " + " ".join(f"{k}={v:.2e}" for k, v in e.items()), flush=True)
    assert e["inv_rms"] <= TOL_F32, e
    for k in ("y", "dx", "dgamma"):
        if k in e:
            assert e[k] <= tol, (label, k, e[k])


# ---- golden fixtures (torch float64) --------------------------------------------

@pytest.mark.parametrize("case", pins.golden_cases(), ids=lambda c: c["name"])
def test_golden_fixture_on_gpu(cuda, case):
    x = np.asarray(case["x"], np.float32).reshape(case["shape"])
    g = None if case["gamma"] is None else np.asarray(case["gamma"], np.float32)
    dy = np.asarray(case["dy"], np.float32).reshape(case["shape"])
    y, inv, dx, dg = gpu_layer(x, g, dy, case["eps"], cuda)
    shp = case["shape"]
    assert row_rel_err(y, np.reshape(case["y"], shp)) <= TOL_F32
    assert vec_rel_err(inv, case["inv_rms"]) <= TOL_F32
    assert dx_rel_err(dx, np.reshape(case["dx"], shp), x, g, dy, case["eps"]) <= TOL_F32
    if case["dgamma"] is not None:
        assert vec_rel_err(dg, case["dgamma"]) <= TOL_F32


# ---- configurations at oracle-friendly sizes --------------------------------------

PARITY_SHAPES = {
    "c1": None,                  # full [4,128,512]
    "c2": (2, 512, 4096),        # 1024 rows of the headline width
    "c3": (1, 512, 8192),        # bf16 outlier distribution, 512 rows
    "c4a": None,                 # full [7,1023,5120]
    "c4b": (65536, 128),         # 65,536 rows of the q/k-norm width
    "c4c": None,                 # full [3,17,13824]
}


@pytest.mark.parametrize("name", sorted(PARITY_SHAPES))
def test_config_parity(cuda, name):
    cfg = configs.CONFIGS[name]
    shape = PARITY_SHAPES[name] or cfg.shape
    print(f"config {name} shape {shape} dtype {cfg.dtype}", flush=True)
    x, g, dy = configs.config_inputs(cfg, shape)
    got = gpu_layer(x, g, dy, cfg.eps, cuda)
    _compare(x, g, dy, cfg.eps, got, f"{name}{shape}")


# ---- every resident launch shape and the looped fallbacks ------------------------

SWEEP_COLS = [1, 3, 4, 8, 10, 16, 32, 64, 100, 128, 256, 512, 1000, 1024, 2048, 3072, 4096,
              5120, 6144, 8192, 12288, 13824, 16384, 20480, 24576, 32768, 40000]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("cols", SWEEP_COLS)
def test_width_sweep(cuda, cols, dtype):
    rows = 37 if cols <= 8192 else 5
    x, g, dy = configs.make_inputs((rows, cols), dtype=dtype, seed=cols)
    got = gpu_layer(x, g, dy, 1e-6, cuda)
    _compare(x, g, dy, 1e-6, got, f"sweep {dtype} {rows}x{cols}")


@pytest.mark.parametrize("rows", [1, 15, 16, 17, 255, 1025, 16385])
def test_row_count_sweep(cuda, rows):
    # ragged row blocks in the backward (16 rows per block minimum)
    x, g, dy = configs.make_inputs((rows, 256), seed=rows)
    got = gpu_layer(x, g, dy, 1e-6, cuda)
    _compare(x, g, dy, 1e-6, got, f"rows {rows}x256")


# ---- modes -----------------------------------------------------------------------

def test_no_gamma_is_ag_rms(cuda):
    x, _, dy = configs.make_inputs((64, 1024), with_gamma=False, seed=3)
    got = gpu_layer(x, None, dy, 1e-5, cuda)
    _compare(x, None, dy, 1e-5, got, "no gamma")


def test_dgamma_not_requested(cuda):
    x, g, dy = configs.make_inputs((64, 1024), seed=4)
    y, inv, dx, dg = gpu_layer(x, g, dy, 1e-6, cuda, want_dgamma=False)
    assert dg is None
    rdx, _ = oracle.bwd(x, g, oracle.fwd(x, g, 1e-6)[1], dy)
    assert dx_rel_err(dx, rdx, x, g, dy, 1e-6) <= TOL_F32


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_accumulate(cuda, dtype):
    x, g, dy = configs.make_inputs((48, 2048), dtype=dtype, seed=5)
    pre_dx, _, _ = configs.make_inputs((48, 2048), dtype=dtype, seed=6, with_gamma=False,
                                       with_dy=False)
    pre_dg = np.linspace(-1, 1, 2048).astype(np.float32)
    y, inv, dx, dg = gpu_layer(x, g, dy, 1e-6, cuda, accumulate=True, pre_dx=pre_dx,
                               pre_dg=pre_dg)
    _, rinv = oracle.fwd(x, g, 1e-6)
    rdx, rdg = oracle.bwd(x, g, rinv, dy, dx=pre_dx, dgamma=pre_dg, accumulate=True)
    # accumulated: compare against the pre-existing gradient's scale as well
    scale = np.maximum(np.max(np.abs(as_f32(rdx)), axis=-1, keepdims=True), 1e-30)
    assert np.max(np.abs(as_f32(dx) - as_f32(rdx)) / scale) <= _tol(x)
    assert vec_rel_err(dg, rdg) <= _tol(x)


def test_misaligned_pointers_take_scalar_path(cuda):
    import torch
    rows, cols = 33, 1024
    x, g, dy = configs.make_inputs((rows, cols), seed=8)
    # views starting one element into a buffer: 4-byte aligned, not 16-byte
    bx = torch.empty(rows * cols + 1, device=cuda)
    bdy = torch.empty(rows * cols + 1, device=cuda)
    by = torch.empty(rows * cols + 1, device=cuda)
    bdx = torch.empty(rows * cols + 1, device=cuda)
    xd = bx[1:].view(rows, cols)
    dyd = bdy[1:].view(rows, cols)
    xd.copy_(torch.from_numpy(x))
    dyd.copy_(torch.from_numpy(dy))
    gd = to_dev(g, cuda)
    assert xd.data_ptr() % 16 != 0
    yv, inv = agk.rmsnorm_fwd(xd, gd, 1e-6, y=by[1:].view(rows, cols))
    dxv, dg = agk.rmsnorm_bwd(xd, gd, inv, dyd, dx=bdx[1:].view(rows, cols))
    torch.cuda.synchronize()
    _compare(x, g, dy, 1e-6, (to_host(yv), to_host(inv), to_host(dxv), to_host(dg)),
             "misaligned")


def test_empty_inputs(cuda):
    import torch
    x = torch.empty(0, 64, device=cuda)
    y, inv = agk.rmsnorm_fwd(x, None, 1e-6)
    assert y.shape == (0, 64)
    dg = torch.full((64,), 7.0, device=cuda)
    agk.rmsnorm_bwd(x, None, inv, x, dgamma=dg)
    torch.cuda.synchronize()
    assert torch.all(dg == 0)            # a fresh gradient of an empty batch is zero
    dg.fill_(7.0)
    agk.rmsnorm_bwd(x, None, inv, x, dgamma=dg, accumulate=True)
    torch.cuda.synchronize()
    assert torch.all(dg == 7.0)          # accumulating nothing leaves it unchanged


def test_workspace_too_small_is_an_error(cuda):
    import torch
    x = torch.randn(64, 256, device=cuda)
    _, inv = agk.rmsnorm_fwd(x, None, 1e-6)
    ws = torch.empty(16, dtype=torch.uint8, device=cuda)
    with pytest.raises(agk.AgkError) as ei:
        agk.rmsnorm_bwd(x, None, inv, x, workspace=ws)
    assert ei.value.status == 3


# ---- full-size configurations: size-independent properties ----------------------

def _full_inputs(cfg, dev):
    """Full-size inputs generated on the GPU (torch's Philox) with cfg's distributions."""
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed(cfg.seed)
    x = torch.randn(cfg.shape, generator=gen, device=dev) * cfg.x_std
    g = torch.rand(cfg.cols, generator=gen, device=dev) + 0.5
    dy = torch.randn(cfg.shape, generator=gen, device=dev)
    if cfg.outlier_p > 0:
        mask = torch.rand(cfg.shape, generator=gen, device=dev) < cfg.outlier_p
        x = torch.where(mask, x * cfg.outlier_scale, x)
    if cfg.dtype == "bf16":
        x, g, dy = x.bfloat16(), g.bfloat16(), dy.bfloat16()
    return x.contiguous(), g.contiguous(), dy.contiguous()


@pytest.mark.slow
@pytest.mark.parametrize("name", ["c2", "c3", "c4a", "c4b"])
def test_full_size_properties(cuda, name):
    import torch
    cfg = configs.CONFIGS[name]
    print(f"full-size {name} {cfg.shape} {cfg.dtype}", flush=True)
    x, g, dy = _full_inputs(cfg, cuda)
    R, D = cfg.rows, cfg.cols
    x2, dy2 = x.view(R, D), dy.view(R, D)
    y, inv = agk.rmsnorm_fwd(x2, g, cfg.eps)
    dx, dg = agk.rmsnorm_bwd(x2, g, inv, dy2)
    torch.cuda.synchronize()

    # 1. sampled rows against the oracle (rows are independent for y, r, dx)
    rng = np.random.default_rng(0)
    rows = np.unique(np.concatenate([[0, R - 1], rng.integers(0, R, 254)]))
    idx = torch.from_numpy(rows).to(cuda)
    xs, dys, gs = to_host(x2[idx].contiguous()), to_host(dy2[idx].contiguous()), to_host(g)
    _compare(xs, gs, dys, cfg.eps, (to_host(y[idx].contiguous()), to_host(inv[idx]),
                                    to_host(dx[idx].contiguous()), None),
             f"{name} sampled rows", check_dg=False)

    # 2. dgamma against an fp64 evaluation of sum_rows dy * x * r on the device
    x64 = x2.double()
    r64 = torch.rsqrt((x64 * x64).mean(dim=1, keepdim=True) + cfg.eps)
    ref = (dy2.double() * x64 * r64).sum(dim=0)
    e = vec_rel_err(to_host(dg), ref.cpu().numpy())
    print(f"[{name}] dgamma vs fp64: {e:.2e}", flush=True)
    assert e <= (TOL_BF16 if cfg.dtype == "bf16" else TOL_F32)

    # 3. the identity sum_j x_j dx_j = dot * eps * r^3, all rows, fp64
    gy = dy2.double() * g.double()
    dot = (gy * x64).sum(dim=1)
    lhs = (x64 * dx.double()).sum(dim=1)
    rhs = dot * cfg.eps * r64.squeeze(1) ** 3
    scale = r64.squeeze(1) * (gy * x64).abs().sum(dim=1)
    ident = float(((lhs - rhs).abs() / scale).max())
    print(f"[{name}] identity residual: {ident:.2e}", flush=True)
    assert ident <= (5e-3 if cfg.dtype == "bf16" else 1e-5)
    del x64, r64, gy

    # 4. dgamma is bit-identical across runs, and dx too
    for _ in range(2):
        dx2, dg2 = agk.rmsnorm_bwd(x2, g, inv, dy2)
        torch.cuda.synchronize()
        assert torch.equal(dg2, dg)
        assert torch.equal(dx2, dx)


# ---- broadcast multiply (the unfused ag::rms(x) * gamma form) ---------------------

@pytest.mark.parametrize("dtype,cols", [("f32", 4096), ("f32", 10), ("bf16", 8192), ("bf16", 7)])
def test_mul_rowbcast(cuda, dtype, cols):
    import torch
    a, b, gy = configs.make_inputs((40, cols), dtype=dtype, seed=cols)
    ad, bd, gyd = to_dev(a, cuda), to_dev(b, cuda), to_dev(gy, cuda)
    y = agk.mul_rowbcast_fwd(ad, bd)
    da, db = agk.mul_rowbcast_bwd(gyd, ad, bd)
    torch.cuda.synchronize()
    af, bf, gf = as_f32(a).astype(np.float64), as_f32(b).astype(np.float64), as_f32(gy).astype(np.float64)
    tol = TOL_BF16 if dtype == "bf16" else TOL_F32
    assert row_rel_err(as_f32(to_host(y)), af * bf) <= tol
    assert row_rel_err(as_f32(to_host(da)), gf * bf) <= tol
    assert vec_rel_err(to_host(db), np.sum(gf * af, axis=0)) <= TOL_F32

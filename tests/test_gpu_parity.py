"""Parity of the HIP path (through the C ABI) with the pinned CPU oracle.

Bars: fp32 storage per-row max|d| / max|ref| <= 1e-5 for y and dx, the same
norm-wise bound for dgamma and, element-wise, each dgamma column against the
sum of its terms' magnitudes; bf16 storage 1e-2; inv_rms 1e-5 relative;
dgamma bit-identical across repeated runs.  Sizes: every configuration at a size the
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
from gpu_util import as_f32, check_on_device, device_inputs, gpu_layer, to_dev, to_host
from tolerances import (TOL_BF16, TOL_F32, dgamma_elem_err, dx_rel_err, row_rel_err,
                        vec_rel_err)

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
        e["dgamma_elem"] = dgamma_elem_err(dg, rdg, as_f32(x), as_f32(dy), rinv)
    print(f"[{label}] " + " ".join(f"{k}={v:.2e}" for k, v in e.items()), flush=True)
    assert e["inv_rms"] <= TOL_F32, e
    for k in ("y", "dx", "dgamma", "dgamma_elem"):
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


@pytest.mark.parametrize("rows", [1, 15, 16, 17, 255, 1023, 1024, 1025, 2047, 2048, 2049,
                                  4097, 16385])
def test_row_count_sweep(cuda, rows):
    # ragged dgamma row blocks: 1 row per block up to 1024 rows, then
    # ceil(rows / 1024) with at least 4 from 2048 rows on
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


@pytest.mark.parametrize("cols", [2048, 1030])   # resident kernel, looped kernel
@pytest.mark.parametrize("flags", [agk.AGK_ACCUM_DX, agk.AGK_ACCUM_DGAMMA])
def test_accumulate_one_output(cuda, cols, flags):
    """dx and dgamma accumulate independently (a tied gamma already holds a
    gradient while x's gradient is fresh, and the other way round)."""
    import torch
    x, g, dy = configs.make_inputs((40, cols), seed=cols + flags)
    xd, gd, dyd = to_dev(x, cuda), to_dev(g, cuda), to_dev(dy, cuda)
    _, inv = agk.rmsnorm_fwd(xd, gd, 1e-6)
    fresh_dx, fresh_dg = agk.rmsnorm_bwd(xd, gd, inv, dyd)
    pre_dx = torch.full_like(xd, 0.25)
    pre_dg = torch.full((cols,), -0.5, device=cuda)
    dx, dg = agk.rmsnorm_bwd(xd, gd, inv, dyd, dx=pre_dx.clone(), dgamma=pre_dg.clone(),
                             accumulate=flags)
    torch.cuda.synchronize()
    if flags == agk.AGK_ACCUM_DX:
        assert torch.equal(dx, pre_dx + fresh_dx) and torch.equal(dg, fresh_dg)
    else:
        assert torch.equal(dx, fresh_dx) and torch.equal(dg, pre_dg + fresh_dg)


@pytest.mark.parametrize("dtype,cols", [("f32", 4096), ("bf16", 8192), ("f32", 1030)])
def test_dgamma_only(cuda, dtype, cols):
    """dx == NULL: only dgamma, bit-identical to the dgamma of a full call."""
    import torch
    x, g, dy = configs.make_inputs((300, cols), dtype=dtype, seed=11)
    xd, gd, dyd = to_dev(x, cuda), to_dev(g, cuda), to_dev(dy, cuda)
    _, inv = agk.rmsnorm_fwd(xd, gd, 1e-6)
    _, full_dg = agk.rmsnorm_bwd(xd, gd, inv, dyd)
    dx, dg = agk.rmsnorm_bwd(xd, gd, inv, dyd, want_dx=False)
    torch.cuda.synchronize()
    assert dx is None
    assert torch.equal(dg, full_dg)


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


# ---- every reachable launch shape ------------------------------------------------

def _plan_cases():
    from plans import reachable_plans
    seen = set()
    cases = []
    for (dt, _direction, _tpr, _nv, _g), reps in sorted(reachable_plans().items()):
        for rows, cols in reps:
            key = ("f32" if dt == agk.AGK_F32 else "bf16", rows, cols)
            if key not in seen:
                seen.add(key)
                cases.append(key)
    return cases


@pytest.mark.parametrize("dtype,rows,cols", _plan_cases(),
                         ids=lambda v: str(v))
def test_every_launch_shape(cuda, dtype, rows, cols):
    """Each resident (lanes, slots, rows-per-workgroup) shape the library can pick,
    at the narrowest and widest width that maps to it, below and above the
    large-batch threshold."""
    dt = agk.AGK_F32 if dtype == "f32" else agk.AGK_BF16
    fp, bp = agk.launch_plan(rows, cols, dt, False), agk.launch_plan(rows, cols, dt, True)
    label = f"{dtype} {rows}x{cols} fwd{(fp['tpr'], fp['nv'], fp['g'])} bwd{(bp['tpr'], bp['nv'], bp['g'])} rpb {bp['rpb']}"
    print(label, flush=True)
    x, g, dy = device_inputs((rows, cols), dtype, rows * 131 + cols, cuda)
    check_on_device(x, g, dy, 1e-6, label, _compare)


# ---- full-size configurations: size-independent properties ----------------------

@pytest.mark.slow
@pytest.mark.parametrize("name", ["c2", "c3", "c4a", "c4b", "c4c"])
def test_full_size_properties(cuda, name):
    cfg = configs.CONFIGS[name]
    print(f"full-size {name} {cfg.shape} {cfg.dtype}", flush=True)
    x, g, dy = device_inputs(cfg.shape, cfg.dtype, cfg.seed, cuda, cfg.x_std, cfg.outlier_p,
                             cfg.outlier_scale)
    R, D = cfg.rows, cfg.cols
    check_on_device(x.view(R, D), g, dy.view(R, D), cfg.eps, name, _compare)


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



@pytest.mark.parametrize("dtype,cols", [("f32", (1 << 24) + 8), ("bf16", (1 << 23) + 24),
                                        ("f32", 1000003)])
def test_mul_one_long_row(cuda, dtype, cols):
    """An equal-shape product reaches the broadcast kernels as one row of numel
    columns (ag::mul with equal shapes); the row is split over many workgroups.
    Products are single roundings of the same operands, so torch's elementwise
    product is bit-exact; db of one row is its gy * a in fp32."""
    import torch
    print(f"mul one row {dtype} {cols}", flush=True)
    gen = torch.Generator(device=cuda)
    gen.manual_seed(cols)
    dt = torch.float32 if dtype == "f32" else torch.bfloat16
    a, b, gy = (torch.randn((1, cols), generator=gen, device=cuda).to(dt) for _ in range(3))
    b = b.view(cols)
    y = agk.mul_rowbcast_fwd(a, b)
    da, db = agk.mul_rowbcast_bwd(gy, a, b)
    torch.cuda.synchronize()
    assert torch.equal(y, a * b)
    assert torch.equal(da, gy * b)
    assert torch.equal(db, (gy.float() * a.float()).view(cols))



@pytest.mark.parametrize("dtype,shape", [("f32", (65536, 4096)), ("bf16", (8192, 11008)),
                                         ("f32", (333, 1001)), ("bf16", (7, 100)),
                                         ("f32", (40, 16392)), ("bf16", (9, 32776)),
                                         ("f32", (1, 4096)), ("f32", (0, 64))])
def test_sum_rows(cuda, dtype, shape):
    """agk_sum_rows (the linear layer's bias gradient): column sums in fp32
    against fp64, bit-identical run to run, accumulate adds exactly the
    fresh sum's rounding onto the old values' (old + new in fp32)."""
    import torch
    R, D = shape
    print(f"sum_rows {dtype} {shape}", flush=True)
    gen = torch.Generator(device=cuda)
    gen.manual_seed(R + D)
    x = torch.randn(shape, generator=gen, device=cuda)
    if dtype == "bf16":
        x = x.bfloat16()
    s1 = agk.sum_rows(x)
    s2 = agk.sum_rows(x)
    old = torch.randn(D, generator=gen, device=cuda)
    s3 = agk.sum_rows(x, out=old.clone(), accumulate=True)
    torch.cuda.synchronize()
    ref = x.double().sum(dim=0)
    assert torch.equal(s1, s2)
    assert torch.equal(s3, old + s1)
    if R:
        assert ((s1.double() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item() <= 1e-6
    else:
        assert torch.count_nonzero(s1).item() == 0


# ---- the unfused layer's two VJPs in one pass (agk_rms_mul_bwd) -------------------

@pytest.mark.parametrize("dtype,shape", [("f32", (40, 4096)), ("f32", (33, 250)),
                                         ("bf16", (96, 8192)), ("bf16", (17, 100)),
                                         ("f32", (24, 16392)), ("bf16", (9, 32776)),
                                         ("f32", (1100, 20480)), ("bf16", (2, 262144)),
                                         ("f32", (65536, 4096)), ("bf16", (16384, 8192)),
                                         # 1-3 steps per workgroup of the three-set
                                         # pipeline, ragged row counts, 1-4 rows per step
                                         ("f32", (300, 4096)), ("bf16", (700, 8192)),
                                         ("f32", (1000, 1024)), ("bf16", (5000, 2048)),
                                         ("f32", (2311, 512))])
def test_rms_mul_bwd(cuda, dtype, shape):
    """Bit-identical to mul_rowbcast_bwd followed by rmsnorm_bwd(gamma=None) on
    the same tensors, overwriting and accumulating; where the oracle is quick,
    dx and dgamma also against the oracle's VJP of the fused layer (the same
    gradients up to the storage rounding of rms(x) and of its gradient)."""
    import torch
    R, D = shape
    print(f"rms_mul_bwd {dtype} {shape}", flush=True)
    x, g, dy = device_inputs(shape, dtype, R * 7 + D, cuda)
    h, inv = agk.rmsnorm_fwd(x, None, 1e-5)
    for acc in (False, True):
        gen = torch.Generator(device=cuda)
        gen.manual_seed(R + D)
        dx0 = torch.randn(shape, generator=gen, device=cuda).to(x.dtype)
        dg0 = torch.randn(D, generator=gen, device=cuda)
        dr, dx, dg = agk.rms_mul_bwd(x, g, inv, dy, dx=dx0.clone() if acc else None,
                                     dgamma=dg0.clone() if acc else None, accumulate=acc)
        dr2, dg2 = agk.mul_rowbcast_bwd(dy, h, g, db=dg0.clone() if acc else None,
                                        accumulate=agk.AGK_ACCUM_DGAMMA if acc else 0)
        dx2, _ = agk.rmsnorm_bwd(x, None, inv, dr2, dx=dx0.clone() if acc else None,
                                 accumulate=agk.AGK_ACCUM_DX if acc else 0, want_dgamma=False)
        torch.cuda.synchronize()
        assert torch.equal(dr, dr2), "dr"
        assert torch.equal(dx, dx2), "dx"
        assert torch.equal(dg, dg2), "dgamma"
    if R * D <= 1 << 20:
        xh, gh, dyh = to_host(x), to_host(g), to_host(dy)
        _, rinv = oracle.fwd(xh, gh, 1e-5)
        rdx, rdg = oracle.bwd(xh, gh, rinv, dyh)
        dr, dx, dg = agk.rms_mul_bwd(x, g, inv, dy)
        torch.cuda.synchronize()
        tol = _tol(xh)
        assert row_rel_err(as_f32(to_host(dx)), as_f32(rdx)) <= tol
        assert vec_rel_err(to_host(dg), rdg) <= tol
        assert row_rel_err(as_f32(to_host(dr)), as_f32(dyh) * as_f32(gh)[None, :]) <= tol

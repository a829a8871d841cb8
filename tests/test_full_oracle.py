"""Every row of the benchmark configurations against the CPU oracle.

The GPU layer (forward, then backward) runs on the configurations' own inputs
at their full sizes; x, gamma and dy go to the host, where the oracle (its
OpenMP build, 16 threads) runs the reference's op sequence over all rows; its
y, inv_rms, dx and dgamma come back to the device, where the errors are taken
in fp64 over every row, a block of rows at a time, with the criteria of
`tolerances` (per-row relative for y, dx against the magnitude of its two
terms, max-relative for inv_rms and dgamma, and each dgamma column against
the sum of its terms' magnitudes).
"""
import os

import numpy as np
import pytest

import cgadimpl_amd as agk
import oracle
from cgadimpl_amd import configs
from gpu_util import device_inputs, to_dev, to_host
from tolerances import TOL_BF16, TOL_F32

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

BLOCK = 4096  # rows per fp64 comparison block


def _row_err(got, ref):
    """max over rows of max|got - ref| / max|ref| (device tensors, one block)."""
    g, r = got.double(), ref.double()
    num = (g - r).abs().amax(dim=1)
    den = r.abs().amax(dim=1)
    if not bool(g.isfinite().all()):
        return float("inf")
    return float(((num / den.clamp_min(1e-300)) * (den > 0) + num * (den == 0)).max())


def _dx_err(got, ref, x, gamma, dy, eps):
    """max over rows of max|got - ref| / (r max|g| + r^3 max|x| |dot| / D)."""
    import torch
    x64 = x.double()
    g64 = dy.double() * gamma.double().unsqueeze(0)
    r = torch.rsqrt((x64 * x64).mean(dim=1) + eps)
    dot = (g64 * x64).sum(dim=1)
    den = r * g64.abs().amax(dim=1) + r ** 3 * x64.abs().amax(dim=1) * dot.abs() / x.shape[1]
    num = (got.double() - ref.double()).abs().amax(dim=1)
    if not bool(got.isfinite().all()):
        return float("inf")
    return float(((num / den.clamp_min(1e-300)) * (den > 0) + num * (den == 0)).max())


def _vec_err(got, ref):
    g, r = got.double(), ref.double()
    den = float(r.abs().max())
    num = float((g - r).abs().max())
    return num / den if den > 0 else num


@pytest.mark.parametrize("name", ["c2", "c3", "c4a", "c4b", "c4c"])
def test_every_row_against_the_oracle(cuda, name):
    import torch
    cfg = configs.CONFIGS[name]
    R, D = cfg.rows, cfg.cols
    print(f"every row {name} {R}x{D} {cfg.dtype}", flush=True)
    x, g, dy = device_inputs(cfg.shape, cfg.dtype, cfg.seed, cuda, cfg.x_std, cfg.outlier_p,
                             cfg.outlier_scale)
    x, dy = x.view(R, D), dy.view(R, D)
    y, inv = agk.rmsnorm_fwd(x, g, cfg.eps)
    dx, dg = agk.rmsnorm_bwd(x, g, inv, dy)
    torch.cuda.synchronize()

    oracle.set_threads(min(16, os.cpu_count() or 1))
    hx, hg, hdy = to_host(x), to_host(g), to_host(dy)
    ry, rinv = oracle.fwd(hx, hg, cfg.eps)
    rdx, rdg = oracle.bwd(hx, hg, rinv, hdy)
    del hx, hg, hdy
    ry, rdx = to_dev(ry, cuda), to_dev(rdx, cuda)
    rinv, rdg = to_dev(rinv, cuda), to_dev(rdg, cuda)
    print(f"[{name}] oracle done", flush=True)

    tol = TOL_BF16 if cfg.dtype == "bf16" else TOL_F32
    e = {"y": 0.0, "dx": 0.0}
    absum = torch.zeros(D, dtype=torch.float64, device=cuda)  # sum_i |dy x r| per column
    for r0 in range(0, R, BLOCK):
        s = slice(r0, min(R, r0 + BLOCK))
        e["y"] = max(e["y"], _row_err(y[s], ry[s]))
        e["dx"] = max(e["dx"], _dx_err(dx[s], rdx[s], x[s], g, dy[s], cfg.eps))
        absum += (dy[s].double() * x[s].double() * rinv[s].double().view(-1, 1)).abs().sum(0)
    e["inv_rms"] = _vec_err(inv, rinv)
    e["dgamma"] = _vec_err(dg, rdg)
    # element-wise: each column against the magnitude of the terms it sums
    num = (dg.double() - rdg.double()).abs()
    e["dgamma_elem"] = float(torch.where(absum > 0, num / absum.clamp_min(1e-300), num).max())
    print(f"[{name}] all {R} rows: " + " ".join(f"{k}={v:.2e}" for k, v in e.items()),
          flush=True)
    for k, v in e.items():
        assert v <= tol, (name, k, v)

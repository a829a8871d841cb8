"""The RMSNorm + linear layer (configuration c5): matmul(rms_norm(x) * gamma, W)
forward and VJP on the GPU kernels, against the CPU oracle's restatement of
the reference graph (bf16 storage, exact products, dW in fp32).

Small shapes run the oracle on every element (including K not a multiple of
64, which takes the staging kernel); the full configuration is checked on
every element against torch's fp32 products of the same bf16 operands and
the oracle's RMSNorm VJP of an independently computed dh.
"""
import numpy as np
import pytest

import cgadimpl_amd as agk
import oracle
from cgadimpl_amd import configs
from gpu_util import as_f32, to_dev, to_host
from tolerances import TOL_BF16, dx_rel_err, row_rel_err, vec_rel_err

pytestmark = pytest.mark.gpu


def _inputs(M, K, N, seed):
    x, g, _ = configs.make_inputs((M, K), dtype="bf16", seed=seed, with_dy=False)
    w, _, _ = configs.make_inputs((K, N), dtype="f32", seed=seed + 1, x_std=0.02,
                                  with_gamma=False, with_dy=False)
    dy, _, _ = configs.make_inputs((M, N), dtype="f32", seed=seed + 2, with_gamma=False,
                                   with_dy=False)
    return x, g, oracle.bf16_encode(w), oracle.bf16_encode(dy)


@pytest.mark.parametrize("M,K,N", [(256, 512, 1024), (200, 520, 264), (64, 4096, 128)])
def test_layer_against_oracle(cuda, M, K, N):
    import torch
    x, g, w, dy = _inputs(M, K, N, seed=M + K + N)
    eps = 1e-5
    ref = oracle.rmsnorm_linear_layer(x, g, w, dy, eps)
    xd, gd, wd, dyd = (to_dev(a, cuda) for a in (x, g, w, dy))
    y, h, inv = agk.rmsnorm_linear_fwd(xd, gd, wd, eps)
    dx, dgamma, dW = agk.rmsnorm_linear_bwd(xd, gd, inv, h, wd, dyd)
    torch.cuda.synchronize()
    errs = {
        "h": row_rel_err(as_f32(to_host(h)), as_f32(ref["h"])),
        "y": row_rel_err(as_f32(to_host(y)), as_f32(ref["y"])),
        "dW": vec_rel_err(to_host(dW), ref["dW"]),
        "dx": dx_rel_err(as_f32(to_host(dx)), as_f32(ref["dx"]), as_f32(x), as_f32(g),
                         as_f32(ref["dh"]), eps),
        "dgamma": vec_rel_err(to_host(dgamma), ref["dgamma"]),
    }
    print(f"[{M}x{K}x{N}] " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    for k, v in errs.items():
        # dW is an fp32 product of bf16 operands: only the accumulation order differs
        assert v <= (1e-5 if k == "dW" else TOL_BF16), (k, v)


def test_layer_full_size(cuda):
    """c5: x [8192, 4096], W [4096, 11008], dy [8192, 11008], bf16, every output
    element checked.  The references are fp32 products computed by torch on
    the GPU (its own GEMM, not this library's) from the same bf16 operands:
    h against the RMSNorm in fp32 (every row), y against h @ W (every row,
    from the layer's own h, which the first check pins), dW against h^T @ dy
    (every element), dx against the CPU oracle's RMSNorm VJP of an
    independent dh = bf16(dy @ W^T) on every row, dgamma against an fp64 sum
    over that independent dh (each column against the sum of its terms'
    magnitudes) and, tighter, over the library's own dh (the GEMM is
    deterministic, so a second call gives the dh the backward used)."""
    import torch
    M, K, N = 8192, 4096, 11008
    gen = torch.Generator(device=cuda)
    gen.manual_seed(5)
    x = torch.randn(M, K, generator=gen, device=cuda).bfloat16()
    g = (torch.rand(K, generator=gen, device=cuda) + 0.5).bfloat16()
    W = (torch.randn(K, N, generator=gen, device=cuda) * 0.02).bfloat16()
    dy = torch.randn(M, N, generator=gen, device=cuda).bfloat16()
    eps = 1e-5
    y, h, inv = agk.rmsnorm_linear_fwd(x, g, W, eps)
    dx, dgamma, dW = agk.rmsnorm_linear_bwd(x, g, inv, h, W, dy)
    torch.cuda.synchronize()

    def rows_err(got, ref):
        """max over rows of max|got - ref| / max|ref| (the row_rel_err form)."""
        num = (got.float() - ref).abs().amax(dim=1)
        return (num / ref.abs().amax(dim=1).clamp_min(1e-30)).max().item()

    xf, gf, Wf, dyf = x.float(), g.float(), W.float(), dy.float()
    rinv = torch.rsqrt(xf.pow(2).mean(dim=1, keepdim=True) + eps)
    e_h = rows_err(h, xf * rinv * gf)
    e_inv = ((inv.view(M, 1) - rinv).abs() / rinv).max().item()
    e_y = rows_err(y, h.float() @ Wf)
    rdW = h.float().t() @ dyf
    e_dW = ((dW - rdW).abs().max() / rdW.abs().max()).item()
    del rdW
    dh_ref = (dyf @ Wf.t()).bfloat16()
    print(f"c5 full size: h {e_h:.2e} inv_rms {e_inv:.2e} y {e_y:.2e} dW {e_dW:.2e}", flush=True)
    assert e_h <= TOL_BF16 and e_inv <= 1e-5 and e_y <= 8e-3 and e_dW <= 1e-5
    # dx on every row: the oracle's VJP of the independent dh.  That dh and the
    # library's can differ by one bf16 unit (2^-8) where their fp32 sums round
    # apart, and both dx are rounded to bf16 (2^-9 each): at most ~7.8e-3 of a
    # row's dx scale, under the bf16 bar
    xs, dhs, gs = to_host(x), to_host(dh_ref), to_host(g)
    _, oinv = oracle.fwd(xs, gs, eps)
    rdx, _ = oracle.bwd(xs, gs, oinv, dhs)
    e_dx = dx_rel_err(as_f32(to_host(dx)), as_f32(rdx), as_f32(xs), as_f32(gs), as_f32(dhs), eps)
    # dgamma: each column against the sum of its terms' magnitudes, over the
    # independent dh; then norm-wise over the library's own dh
    terms = dh_ref.double() * x.double() * inv.double().view(M, 1)
    rdg = terms.sum(dim=0)
    e_dg_ind = ((dgamma.double() - rdg).abs() / terms.abs().sum(dim=0)).max().item()
    del terms
    dh_own = agk.gemm_bf16(dy, W, trans_b=True)
    rdg_own = (dh_own.double() * x.double() * inv.double().view(M, 1)).sum(dim=0)
    e_dg = ((dgamma.double() - rdg_own).abs().max() / rdg_own.abs().max()).item()
    print(f"  dx {e_dx:.2e} dgamma (independent dh, per column) {e_dg_ind:.2e} "
          f"(own dh) {e_dg:.2e}", flush=True)
    assert e_dx <= TOL_BF16 and e_dg_ind <= TOL_BF16 and e_dg <= 1e-5
    # determinism of the whole backward
    dx2, dg2, dW2 = agk.rmsnorm_linear_bwd(x, g, inv, h, W, dy)
    torch.cuda.synchronize()
    assert torch.equal(dx, dx2) and torch.equal(dgamma, dg2) and torch.equal(dW, dW2)

"""The RMSNorm + linear layer (configuration c5): matmul(rms_norm(x) * gamma, W)
forward and VJP on the GPU kernels, against the CPU oracle's restatement of
the reference graph (bf16 storage, exact products, dW in fp32).

Small shapes run the oracle on every element (including K not a multiple of
64, which takes the staging kernel); the full configuration is checked on
sampled rows and columns and through the RMSNorm VJP of the GPU's own dh.
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
    """c5: x [8192, 4096], W [4096, 11008], dy [8192, 11008], bf16."""
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
    rows = torch.randint(0, M, (48,), generator=gen, device=cuda)
    ry = h[rows].float() @ W.float()
    assert ((y[rows].float() - ry).abs().max() / ry.abs().max()).item() <= 8e-3
    cols = torch.randint(0, K, (16,), generator=gen, device=cuda)
    rdW = h[:, cols].float().t() @ dy.float()
    assert ((dW[cols] - rdW).abs().max() / rdW.abs().max()).item() <= 1e-5
    # dx, dgamma: the RMSNorm VJP of dh = dy W^T, on sampled rows against the oracle
    dh = (dy[rows].float() @ W.float().t()).bfloat16()
    xs, dhs = to_host(x[rows].contiguous()), to_host(dh)
    _, rinv = oracle.fwd(xs, to_host(g), eps)
    rdx, _ = oracle.bwd(xs, to_host(g), rinv, dhs)
    e = dx_rel_err(as_f32(to_host(dx[rows].contiguous())), as_f32(rdx), as_f32(xs),
                   as_f32(to_host(g)), as_f32(dhs), eps)
    assert e <= TOL_BF16, e
    # dgamma over all 8192 rows against an fp64 reduction of the same dh (the
    # GEMM is deterministic, so a second dh = dy W^T is the one the backward
    # used): dgamma[j] = sum_i dh[i, j] * x[i, j] * inv_rms[i]
    dh_all = agk.gemm_bf16(dy, W, trans_b=True)
    rdg = (dh_all.double() * x.double() * inv.double().view(M, 1)).sum(dim=0)
    e = ((dgamma.double() - rdg).abs().max() / rdg.abs().max()).item()
    assert e <= 1e-5, e
    # determinism of the whole backward
    dx2, dg2, dW2 = agk.rmsnorm_linear_bwd(x, g, inv, h, W, dy)
    torch.cuda.synchronize()
    assert torch.equal(dx, dx2) and torch.equal(dgamma, dg2) and torch.equal(dW, dW2)

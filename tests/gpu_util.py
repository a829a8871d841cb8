"""Host <-> device plumbing for the GPU tests (numpy arrays in, numpy out)."""
from __future__ import annotations

import numpy as np

import cgadimpl_amd as agk


def to_dev(a, dev):
    import torch
    if a is None:
        return None
    if a.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def to_host(t):
    import torch
    if t is None:
        return None
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def gpu_layer(x, gamma, dy, eps, dev, accumulate=False, pre_dx=None, pre_dg=None,
              want_dgamma=True):
    """Runs fwd + bwd through the C ABI; returns numpy (y, inv_rms, dx, dgamma)."""
    import torch
    xd, gd, dyd = to_dev(x, dev), to_dev(gamma, dev), to_dev(dy, dev)
    y, inv = agk.rmsnorm_fwd(xd, gd, eps)
    dx = to_dev(pre_dx, dev) if pre_dx is not None else None
    dg = to_dev(pre_dg, dev) if pre_dg is not None else None
    dx, dg = agk.rmsnorm_bwd(xd, gd, inv, dyd, dx=dx, dgamma=dg, accumulate=accumulate,
                             want_dgamma=want_dgamma)
    torch.cuda.synchronize()
    return to_host(y), to_host(inv), to_host(dx), to_host(dg)


def as_f32(a):
    if a is None:
        return None
    if a.dtype == np.uint16:
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.astype(np.float32)


def device_inputs(shape, dtype, seed, dev, x_std=1.0, outlier_p=0.0, outlier_scale=1.0):
    """Inputs generated on the GPU (torch's Philox) with the configurations'
    distributions: x ~ N(0, x_std^2) with outliers, gamma ~ U(0.5, 1.5), dy ~ N(0, 1)."""
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    cols = shape[-1]
    x = torch.randn(shape, generator=gen, device=dev) * x_std
    g = torch.rand(cols, generator=gen, device=dev) + 0.5
    dy = torch.randn(shape, generator=gen, device=dev)
    if outlier_p > 0:
        mask = torch.rand(shape, generator=gen, device=dev) < outlier_p
        x = torch.where(mask, x * outlier_scale, x)
        del mask
    if dtype == "bf16":
        x, g, dy = x.bfloat16(), g.bfloat16(), dy.bfloat16()
    return x.contiguous(), g.contiguous(), dy.contiguous()


def check_on_device(x, g, dy, eps, label, compare, sample=254, tol=None):
    """Runs the layer on device tensors and checks size-independent properties.

    1. sampled rows (all rows when there are few) against the CPU oracle
       through `compare` (rows are independent for y, inv_rms and dx);
    2. dgamma against an fp64 evaluation of sum_rows dy * x * r on the device;
    3. the identity sum_j x_j dx_j = dot * eps * r^3 on every row (fp64);
    4. dx and dgamma bit-identical across repeated backward calls.
    """
    import torch
    from tolerances import TOL_BF16, TOL_F32, vec_rel_err
    bf16 = x.dtype == torch.bfloat16
    tol = tol or (TOL_BF16 if bf16 else TOL_F32)
    R, D = x.shape
    y, inv = agk.rmsnorm_fwd(x, g, eps)
    dx, dg = agk.rmsnorm_bwd(x, g, inv, dy)
    torch.cuda.synchronize()

    rng = np.random.default_rng(R * 7919 + D)
    if R <= sample + 2:
        rows = np.arange(R)
    else:
        rows = np.unique(np.concatenate([[0, R - 1], rng.integers(0, R, sample)]))
    idx = torch.from_numpy(rows).to(x.device)
    compare(to_host(x[idx].contiguous()), to_host(g), to_host(dy[idx].contiguous()), eps,
            (to_host(y[idx].contiguous()), to_host(inv[idx]), to_host(dx[idx].contiguous()),
             None), f"{label} sampled rows", check_dg=False)

    x64 = x.double()
    r64 = torch.rsqrt((x64 * x64).mean(dim=1, keepdim=True) + eps)
    ref = (dy.double() * x64 * r64).sum(dim=0)
    e = vec_rel_err(to_host(dg), ref.cpu().numpy())
    print(f"[{label}] dgamma vs fp64: {e:.2e}", flush=True)
    assert e <= tol, (label, "dgamma", e)

    gy = dy.double() * g.double()
    dot = (gy * x64).sum(dim=1)
    lhs = (x64 * dx.double()).sum(dim=1)
    rhs = dot * eps * r64.squeeze(1) ** 3
    scale = r64.squeeze(1) * (gy * x64).abs().sum(dim=1)
    ident = float(((lhs - rhs).abs() / scale).max())
    print(f"[{label}] identity residual: {ident:.2e}", flush=True)
    assert ident <= (5e-3 if bf16 else 1e-5), (label, "identity", ident)
    del x64, r64, gy, dot, lhs, rhs, scale, ref

    for _ in range(2):
        dx2, dg2 = agk.rmsnorm_bwd(x, g, inv, dy)
        torch.cuda.synchronize()
        assert torch.equal(dg2, dg), (label, "dgamma not deterministic")
        assert torch.equal(dx2, dx), (label, "dx not deterministic")

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

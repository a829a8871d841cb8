"""agk_rmsnorm_bwd_noalloc: the backward without a workspace, against agk_rmsnorm_bwd.

The no-alloc entry point runs the same kernels with the dgamma partial rows in
the library's per-device scratch array instead of a caller workspace, so its
outputs must equal agk_rmsnorm_bwd's bit for bit.  The calls follow one
another on one stream, each smaller than the one before, so a later call
reads a scratch array that still holds the previous call's partial rows.
"""
import ctypes

import numpy as np
import pytest

import cgadimpl_amd as agk
from gpu_util import device_inputs, to_host

pytestmark = pytest.mark.gpu


def _noalloc(x, gamma, inv, dy, dx, dg, accumulate, stream):
    rows, cols = x.shape
    dt = agk.AGK_F32 if x.dtype.is_floating_point and x.element_size() == 4 else agk.AGK_BF16
    return agk.lib().agk_rmsnorm_bwd_noalloc(
        x.data_ptr(), gamma.data_ptr() if gamma is not None else None, inv.data_ptr(),
        dy.data_ptr(), dx.data_ptr() if dx is not None else None,
        dg.data_ptr() if dg is not None else None, rows, cols, dt, accumulate,
        stream.cuda_stream)


def _pair(cuda, rows, cols, dtype, accumulate, seed):
    """Both entry points on the same inputs; returns (reference, no-alloc) outputs."""
    import torch
    x, g, dy = device_inputs((rows, cols), dtype, seed, cuda)
    _, inv = agk.rmsnorm_fwd(x, g, 1e-6)
    stream = torch.cuda.current_stream()
    gen = torch.Generator(device=cuda)
    gen.manual_seed(seed + 1)
    dx0 = torch.randn((rows, cols), generator=gen, device=cuda).to(x.dtype)
    dg0 = torch.randn(cols, generator=gen, device=cuda)
    ref_dx, ref_dg = dx0.clone(), dg0.clone()
    agk.rmsnorm_bwd(x, g, inv, dy, dx=ref_dx, dgamma=ref_dg, accumulate=accumulate,
                    stream=stream)
    na_dx, na_dg = dx0.clone(), dg0.clone()
    rc = _noalloc(x, g, inv, dy, na_dx, na_dg, accumulate, stream)
    assert rc == 0, agk.STATUS.get(rc, rc)
    torch.cuda.synchronize()
    return (to_host(ref_dx), to_host(ref_dg)), (to_host(na_dx), to_host(na_dg))


# (rows, cols, dtype, accumulate bits): each call smaller than the one before it;
# the register-resident kernel (256 partial rows), the split path for wide rows
# (partial rows, segment sums and coefficients; then one row block writing
# dgamma directly), the one-pass kernel for 256+ rows of up to 32768 columns, the looped kernel (unaligned rows, one partial row per row
# block) and the few-rows kernel (no partials).
CALLS = [
    (16384, 4096, "f32", 0),
    (300, 65536, "f32", agk.AGK_ACCUM_ALL),
    (512, 24576, "bf16", agk.AGK_ACCUM_DGAMMA),
    (1000, 1536, "bf16", agk.AGK_ACCUM_ALL),
    (600, 1001, "f32", agk.AGK_ACCUM_DGAMMA),
    (51, 13824, "f32", 0),
    (1, 131072, "bf16", agk.AGK_ACCUM_DX),
]


def test_noalloc_matches_workspace_backward_across_calls(cuda):
    for i, (rows, cols, dtype, acc) in enumerate(CALLS):
        print(f"noalloc call {i}: {rows}x{cols} {dtype} accumulate={acc}", flush=True)
        (rdx, rdg), (ndx, ndg) = _pair(cuda, rows, cols, dtype, acc, seed=100 + i)
        assert np.array_equal(rdx.view(np.uint8), ndx.view(np.uint8)), f"dx differs, call {i}"
        assert np.array_equal(rdg.view(np.uint8), ndg.view(np.uint8)), f"dgamma differs, call {i}"


# dx only (dgamma NULL) on wide rows: the split path with only the row
# statistics in the scratch array, as agk_rmsnorm_bwd takes it with a workspace;
# then a resident width, which needs no scratch at all.
DX_ONLY_CALLS = [
    (300, 65536, "f32", 0),
    (1, 131072, "bf16", agk.AGK_ACCUM_DX),
    (512, 4096, "f32", 0),
]


def test_noalloc_dx_only_matches_workspace_backward(cuda):
    import torch
    for i, (rows, cols, dtype, acc) in enumerate(DX_ONLY_CALLS):
        print(f"noalloc dx-only call {i}: {rows}x{cols} {dtype} accumulate={acc}", flush=True)
        x, g, dy = device_inputs((rows, cols), dtype, 300 + i, cuda)
        _, inv = agk.rmsnorm_fwd(x, g, 1e-6)
        stream = torch.cuda.current_stream()
        gen = torch.Generator(device=cuda)
        gen.manual_seed(400 + i)
        dx0 = torch.randn((rows, cols), generator=gen, device=cuda).to(x.dtype)
        ref = dx0.clone()
        agk.rmsnorm_bwd(x, g, inv, dy, dx=ref, want_dgamma=False, accumulate=acc, stream=stream)
        got = dx0.clone()
        rc = _noalloc(x, g, inv, dy, got, None, acc, stream)
        assert rc == 0, agk.STATUS.get(rc, rc)
        torch.cuda.synchronize()
        assert np.array_equal(to_host(ref).view(np.uint8), to_host(got).view(np.uint8)), \
            f"dx differs, dx-only call {i}"


def test_noalloc_rejects_partials_beyond_the_scratch_array(cuda):
    import torch
    rows, cols = 300, 40001  # looped kernel: 300 row blocks x 40001 fp32 partials = 48 MB
    x = torch.zeros((rows, cols), dtype=torch.float32, device=cuda)
    inv = torch.ones(rows, dtype=torch.float32, device=cuda)
    dg = torch.zeros(cols, dtype=torch.float32, device=cuda)
    rc = _noalloc(x, None, inv, x, None, dg, 0, torch.cuda.current_stream())
    assert rc == 3  # AGK_EWORKSPACE, before any launch
    torch.cuda.synchronize()

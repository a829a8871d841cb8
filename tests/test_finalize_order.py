"""dgamma's fixed summation order, checked bit for bit from the partial rows.

After a backward call the caller's workspace still holds the fp32 partial
rows the finalize summed (at its start, or after the wide paths' row
statistics), so the host can redo the finalize in float64 in the
documented order and compare every bit of dgamma:
  more than 64 partial rows: split s (of 64) adds rows s, s+64, s+128, ... in
  increasing order from +0.0, then the split sums are added in split order;
  at most 64: the rows added in increasing order from +0.0 (the same sum: each
  split then holds at most one row);
and with accumulation, the fp32 sum old + float(total).  Covers the resident
kernel (256 partial rows), the looped kernel (unaligned rows: one partial row
per row block, few and many), the one-pass kernel for rows of up to 32768
columns (256 partial rows) and the team kernel for wider rows (one partial
row per team).
"""
import numpy as np
import pytest

import cgadimpl_amd as agk
from gpu_util import device_inputs

pytestmark = pytest.mark.gpu

SPLITS = 64


def _r256(b):
    return (b + 255) // 256 * 256


def _finalize_f64(parts):
    """The documented order, in numpy float64 (vectorised over columns only)."""
    nblk = parts.shape[0]
    p = parts.astype(np.float64)
    if nblk <= SPLITS:
        tot = np.zeros(parts.shape[1])
        for b in range(nblk):
            tot = tot + p[b]
        return tot
    split = np.zeros((SPLITS, parts.shape[1]))
    for s in range(SPLITS):
        for b in range(s, nblk, SPLITS):
            split[s] = split[s] + p[b]
    tot = split[0].copy()
    for s in range(1, SPLITS):
        tot = tot + split[s]
    return tot


@pytest.mark.parametrize("dtype,rows,cols", [
    ("f32", 33, 1030),       # looped, 33 partial rows (at most 64), unaligned columns
    ("f32", 300, 1030),      # looped, 300 partial rows
    ("bf16", 70, 1001),      # looped, 70 partial rows
    ("f32", 8, 262144),      # team kernel, 8 teams
    ("f32", 300, 65536),     # team kernel, 64 teams (the boundary)
    ("bf16", 1030, 65544),   # team kernel, 65 teams
    ("f32", 1100, 20480),    # one pass, 256 partial rows
    ("f32", 4096, 4096),     # resident, 256 partial rows
], ids=str)
@pytest.mark.parametrize("accumulate", [False, True])
def test_dgamma_is_the_documented_sum_of_the_partial_rows(cuda, dtype, rows, cols, accumulate):
    import torch
    dt = agk.AGK_F32 if dtype == "f32" else agk.AGK_BF16
    plan = agk.launch_plan(rows, cols, dt, True)
    nblk = plan["nblk"]
    assert nblk > 0, f"no partial rows for this shape: {plan}"
    print(f"{dtype} {rows}x{cols} plan {plan} accumulate={accumulate}", flush=True)
    x, g, dy = device_inputs((rows, cols), dtype, rows + cols, cuda)
    _, inv = agk.rmsnorm_fwd(x, g, 1e-6)
    ws = torch.zeros(agk.rmsnorm_bwd_workspace_bytes(rows, cols), dtype=torch.uint8,
                     device=cuda)
    pre = torch.linspace(-3.0, 3.0, cols, device=cuda)
    dg = pre.clone()
    # misaligned (looped) shapes: the plan assumes aligned pointers, which
    # torch's allocations are; unaligned columns are what make them looped
    agk.rmsnorm_bwd(x, g, inv, dy, dgamma=dg, workspace=ws, accumulate=accumulate)
    torch.cuda.synchronize()
    # the split path and the team kernel keep their row statistics (8-byte
    # segment slots, then the coefficients, each region 256-byte aligned)
    # ahead of the partial rows
    off = 0
    if (plan["tpr"] == 0 and plan["nv"] > 0) or (plan["tpr"] > 0 and plan["g"] == 0):
        off = _r256(rows * -(-cols // 4096) * 8) + _r256(rows * 4)
    parts = ws[off: off + nblk * cols * 4].view(torch.float32).view(nblk, cols).cpu().numpy()
    tot = _finalize_f64(parts).astype(np.float32)
    want = (pre.cpu().numpy() + tot).astype(np.float32) if accumulate else tot
    got = dg.cpu().numpy()
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, (f"{bad.size} columns differ, first {bad[:5]}: "
                           f"{got[bad[:5]]} vs {want[bad[:5]]}")

"""Rows wider than the register-resident shapes: two forward paths -- the
split forward (several workgroups per row for the row statistics, then
row-chunk scaling) and, given a workspace, the team forward (a row over
several workgroups that exchange their segment sums: x read once) -- and
three backward paths: from 256 rows of at most 32768 columns the one-pass
kernel (x and dy in registers, dgamma in LDS); other aligned rows of up to
1M columns the team kernel (a row over several workgroups that exchange
their segment sums through the workspace); wider rows the split path (row
statistics, then row-block x column-chunk tiles for dx and dgamma).

Against the CPU oracle (fp64 accumulation) at sizes it finishes in seconds,
through the size-independent properties at full sizes, bit-identical across
runs, with accumulation and the one-output modes bit-identical to the full
call, and the fallbacks that keep the one-workgroup-per-row kernels (an
in-place forward, a dx-only call without workspace, rows that are not whole
16-byte slots) within the same bars.
"""
import ctypes

import numpy as np
import pytest

import cgadimpl_amd as agk
import oracle
from cgadimpl_amd import configs
from gpu_util import as_f32, check_on_device, device_inputs, gpu_layer, to_dev, to_host
from tolerances import TOL_BF16, TOL_F32, dx_rel_err, row_rel_err, vec_rel_err

pytestmark = pytest.mark.gpu


def _tol(x):
    return TOL_BF16 if x.dtype == np.uint16 else TOL_F32


def _compare(x, gamma, dy, eps, got, label, check_dg=True):
    y, inv, dx, dg = got
    ry, rinv = oracle.fwd(x, gamma, eps)
    rdx, rdg = oracle.bwd(x, gamma, rinv, dy)
    tol = _tol(x)
    e = {"y": row_rel_err(as_f32(y), as_f32(ry)), "inv_rms": vec_rel_err(inv, rinv),
         "dx": dx_rel_err(as_f32(dx), as_f32(rdx), as_f32(x), as_f32(gamma), as_f32(dy), eps)}
    if check_dg:
        e["dgamma"] = vec_rel_err(dg, rdg)
    print(f"[{label}] " + " ".join(f"{k}={v:.2e}" for k, v in e.items()), flush=True)
    assert e["inv_rms"] <= TOL_F32, (label, e)
    for k in ("y", "dx", "dgamma"):
        if k in e:
            assert e[k] <= tol, (label, k, e[k])


def _dt(dtype):
    return agk.AGK_F32 if dtype == "f32" else agk.AGK_BF16


# (dtype, rows, cols): few very long rows (one row block: dgamma written by the
# tiles), ragged last segment and chunk, and enough rows for several row
# blocks (partial rows + finalize); from 256 rows of at most 32768 columns the
# one-pass backward (x and dy in registers, dgamma in LDS).
WIDE_CASES = [
    ("f32", 8, 262144),
    ("f32", 1, 1 << 20),
    ("f32", 3, 40000),
    ("f32", 2, 131076),
    ("bf16", 3, 65544),
    ("bf16", 5, 131080),
    ("bf16", 7, 24576),
    ("f32", 300, 65536),
    ("bf16", 1030, 40000),
    ("f32", 1100, 40000),
    ("bf16", 1030, 65544),
    ("f32", 255, 32768),
    ("f32", 1100, 20480),
    ("f32", 256, 16388),
    ("f32", 300, 32768),
    ("bf16", 257, 16392),
    ("bf16", 1024, 24576),
    ("bf16", 300, 32768),
]


def _one_pass(rows, cols):
    return rows >= 256 and cols <= 32768


def _team(rows, cols):
    return not _one_pass(rows, cols) and rows >= 4 and -(-cols // 4096) <= 256


@pytest.mark.parametrize("dtype,rows,cols", WIDE_CASES, ids=str)
def test_wide_parity(cuda, dtype, rows, cols):
    fp = agk.launch_plan(rows, cols, _dt(dtype), False)
    bp = agk.launch_plan(rows, cols, _dt(dtype), True)
    label = f"wide {dtype} {rows}x{cols} fwd {fp} bwd {bp}"
    print(label, flush=True)
    if _one_pass(rows, cols):
        assert bp["tpr"] == 1024 and bp["nv"] == (8 if dtype == "f32" else 4), \
            "backward should take the one-pass kernel"
    elif _team(rows, cols):
        assert bp["tpr"] > 0 and bp["g"] == 0, "backward should take the team kernel"
    else:
        assert bp["tpr"] == 0 and bp["nv"] > 0, "backward should take the split path"
    if fp["tpr"] == 0:
        assert fp["nv"] > 0, "forward should take the split path"
    x, g, dy = configs.make_inputs((rows, cols), dtype=dtype, seed=rows * 7 + cols)
    got = gpu_layer(x, g, dy, 1e-6, cuda)
    _compare(x, g, dy, 1e-6, got, label)


@pytest.mark.slow
@pytest.mark.parametrize("dtype,rows,cols", [("f32", 4096, 32768), ("bf16", 1024, 65536),
                                             ("f32", 64, 1 << 21), ("bf16", 16384, 20480)],
                         ids=str)
def test_wide_full_size_properties(cuda, dtype, rows, cols):
    label = f"wide {dtype} {rows}x{cols}"
    print(label, flush=True)
    x, g, dy = device_inputs((rows, cols), dtype, rows + cols, cuda)
    check_on_device(x, g, dy, 1e-6, label, _compare, sample=16)


# Team kernel shapes: many rows (more rows than teams), one row per team,
# ragged last segment, the widest rows it takes (256 segments), bf16 parts of
# two segments with an odd segment count, fp32 parts of two segments (gamma
# in LDS) chosen by the width (64 one-segment parts) and by the rows per team
# (with a ragged last segment).
TEAM_CASES = [("f32", 300, 65536), ("bf16", 100, 131072), ("f32", 4, 40000),
              ("bf16", 5, 131080), ("f32", 4, 1 << 20), ("bf16", 70, 36864),
              ("f32", 9, 16388), ("f32", 40, 262144), ("f32", 1700, 40004)]


@pytest.mark.parametrize("dtype,rows,cols", TEAM_CASES, ids=str)
@pytest.mark.parametrize("with_gamma", [True, False], ids=["gamma", "no_gamma"])
def test_team_against_split_and_recompute(cuda, dtype, rows, cols, with_gamma):
    """The team kernel against the split path on the same inputs (the team
    switched off): dx bit-identical, since both add the same 4096-column
    segment sums in the same order and apply the same per-element formula;
    dgamma within the oracle's bar of each other (different partial rows: one
    per team against one per row block).  With every wait cut to its first
    look (wait limit 0, so the workgroups recompute the sums they do not find
    yet), dx and dgamma bit-identical to the default: a recomputed sum is the
    published one.  Both against the oracle."""
    import torch
    x, g, dy = configs.make_inputs((rows, cols), dtype=dtype, with_gamma=with_gamma,
                                   seed=rows * 5 + cols)
    xd, dyd = to_dev(x, cuda), to_dev(dy, cuda)
    gd = to_dev(g, cuda) if with_gamma else None
    _, inv = agk.rmsnorm_fwd(xd, gd, 1e-6)
    plan = agk.launch_plan(rows, cols, _dt(dtype), True)
    print(f"team {dtype} {rows}x{cols} gamma={with_gamma} plan {plan}", flush=True)
    assert plan["tpr"] > 0 and plan["g"] == 0
    team_dx, team_dg = agk.rmsnorm_bwd(xd, gd, inv, dyd)
    prev = agk.set_team_backward(0)
    try:
        split_dx, split_dg = agk.rmsnorm_bwd(xd, gd, inv, dyd)
    finally:
        agk.set_team_backward(prev)
    prev = agk.set_exchange_wait_limit(0)
    try:
        rec_dx, rec_dg = agk.rmsnorm_bwd(xd, gd, inv, dyd)
    finally:
        agk.set_exchange_wait_limit(prev)
    torch.cuda.synchronize()
    assert torch.equal(team_dx, split_dx)
    assert torch.equal(rec_dx, team_dx)
    assert torch.equal(rec_dg, team_dg)
    _, rinv = oracle.fwd(x, g if with_gamma else None, 1e-6)
    rdx, rdg = oracle.bwd(x, g if with_gamma else None, rinv, dy)
    e_team = vec_rel_err(to_host(team_dg), rdg)
    e_split = vec_rel_err(to_host(split_dg), rdg)
    e_dx = dx_rel_err(as_f32(to_host(team_dx)), as_f32(rdx), as_f32(x),
                      as_f32(g) if with_gamma else None, as_f32(dy), 1e-6)
    print(f"  dx {e_dx:.2e} dgamma team {e_team:.2e} split {e_split:.2e}", flush=True)
    assert e_dx <= _tol(x) and e_team <= TOL_F32 and e_split <= TOL_F32


# Team forward shapes (agk_rmsnorm_fwd_ws): more rows than teams, a ragged
# last segment (fp32) and an odd segment count (bf16 parts of four), the
# widest rows it takes (256 segments), the fewest rows it takes (4), fp32
# parts of four segments (gamma in LDS) chosen by the rows per team and by
# the width.
FWD_TEAM_CASES = [("f32", 600, 40000), ("f32", 7, 50000), ("f32", 4, 1 << 20),
                  ("f32", 300, 65536), ("bf16", 100, 131072), ("bf16", 5, 131080),
                  ("bf16", 6, 70008), ("bf16", 4, 1 << 20), ("f32", 256, 65536),
                  ("f32", 40, 262144)]


@pytest.mark.parametrize("dtype,rows,cols", FWD_TEAM_CASES, ids=str)
@pytest.mark.parametrize("with_gamma", [True, False], ids=["gamma", "no_gamma"])
def test_team_forward_against_split_and_recompute(cuda, dtype, rows, cols, with_gamma):
    """agk_rmsnorm_fwd_ws (the team kernel, x read once) against
    agk_rmsnorm_fwd (the split path, x read twice) on the same inputs: y and
    inv_rms bit-identical, since both add the same 4096-column segment sums in
    the same order and apply the same per-element formula.  The workspace
    starts with every flag set (its contents on entry must not matter).  With
    every wait cut to its first look (wait limit 0: the workgroups recompute
    the sums they do not find yet) bit-identical again.  Against the oracle."""
    import torch
    x, g, _ = configs.make_inputs((rows, cols), dtype=dtype, with_gamma=with_gamma,
                                  with_dy=False, seed=rows * 11 + cols)
    xd = to_dev(x, cuda)
    gd = to_dev(g, cuda) if with_gamma else None
    plan = agk.launch_plan(rows, cols, _dt(dtype), False, fwd_workspace=True)
    print(f"team fwd {dtype} {rows}x{cols} gamma={with_gamma} plan {plan}", flush=True)
    assert plan["tpr"] > 0 and plan["g"] == 0
    ws = torch.full((agk.rmsnorm_fwd_workspace_bytes(rows, cols),), 255, dtype=torch.uint8,
                    device=cuda)
    team_y, team_inv = agk.rmsnorm_fwd(xd, gd, 1e-6, workspace=ws)
    split_y, split_inv = agk.rmsnorm_fwd(xd, gd, 1e-6)
    prev = agk.set_exchange_wait_limit(0)
    try:
        rec_y, rec_inv = agk.rmsnorm_fwd(xd, gd, 1e-6, workspace=ws)
    finally:
        agk.set_exchange_wait_limit(prev)
    torch.cuda.synchronize()
    assert torch.equal(team_inv, split_inv) and torch.equal(team_y, split_y)
    assert torch.equal(rec_inv, team_inv) and torch.equal(rec_y, team_y)
    ry, rinv = oracle.fwd(x, g if with_gamma else None, 1e-6)
    ey = row_rel_err(as_f32(to_host(team_y)), as_f32(ry))
    ei = vec_rel_err(to_host(team_inv), rinv)
    print(f"  y {ey:.2e} inv_rms {ei:.2e}", flush=True)
    assert ey <= _tol(x) and ei <= TOL_F32


@pytest.mark.parametrize("rows,cols,in_place", [(3, 65536, False), (4, 65536, True),
                                                (4, 40002, False), (5, 16384, False)],
                         ids=str)
def test_team_forward_fallbacks(cuda, rows, cols, in_place):
    """agk_rmsnorm_fwd_ws where its team kernel does not apply -- fewer than 4
    rows, y == x, rows that are not whole 16-byte slots, rows one workgroup
    holds -- runs agk_rmsnorm_fwd's kernels: bit-identical to it."""
    import torch
    x, g, _ = configs.make_inputs((rows, cols), with_dy=False, seed=cols + rows)
    xd, gd = to_dev(x, cuda), to_dev(g, cuda)
    ws = torch.empty(max(agk.rmsnorm_fwd_workspace_bytes(rows, cols), 8), dtype=torch.uint8,
                     device=cuda)
    if in_place:
        a, b = xd.clone(), xd.clone()
        ya, inva = agk.rmsnorm_fwd(a, gd, 1e-6, y=a, workspace=ws)
        yb, invb = agk.rmsnorm_fwd(b, gd, 1e-6, y=b)
    else:
        ya, inva = agk.rmsnorm_fwd(xd, gd, 1e-6, workspace=ws)
        yb, invb = agk.rmsnorm_fwd(xd, gd, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(ya, yb) and torch.equal(inva, invb)


def test_team_kernels_on_two_streams_at_once(cuda):
    """Team kernels of two calls running at once on two streams (default
    priority), whose grids together exceed the 512 workgroups the GPU holds
    at the kernels' register use: some teams wait on members that are not
    resident and recompute the sums they miss.  Every output bit-identical to
    the same calls made one after the other."""
    import torch
    rows, cols = 1024, 65536
    a = device_inputs((rows, cols), "f32", 91, cuda)
    b = device_inputs((rows, cols), "bf16", 92, cuda)
    _, inv_a = agk.rmsnorm_fwd(a[0], a[1], 1e-6)
    _, inv_b = agk.rmsnorm_fwd(b[0], b[1], 1e-6)
    torch.cuda.synchronize()
    # one after the other
    ref_fa = agk.rmsnorm_fwd(a[0], a[1], 1e-6, workspace=None)
    ref_ba = agk.rmsnorm_bwd(a[0], a[1], inv_a, a[2])
    ref_fb = agk.rmsnorm_fwd(b[0], b[1], 1e-6, workspace=None)
    ref_bb = agk.rmsnorm_bwd(b[0], b[1], inv_b, b[2])
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    ws = [torch.empty(agk.rmsnorm_bwd_workspace_bytes(rows, cols), dtype=torch.uint8, device=cuda)
          for _ in range(2)]
    fws = [torch.empty(agk.rmsnorm_fwd_workspace_bytes(rows, cols), dtype=torch.uint8,
                       device=cuda) for _ in range(2)]
    out = {}
    for rep in range(3):
        with torch.cuda.stream(s1):
            out["fa"] = agk.rmsnorm_fwd(a[0], a[1], 1e-6, workspace=fws[0], stream=s1)
            out["ba"] = agk.rmsnorm_bwd(a[0], a[1], inv_a, a[2], workspace=ws[0], stream=s1)
        with torch.cuda.stream(s2):
            out["bb"] = agk.rmsnorm_bwd(b[0], b[1], inv_b, b[2], workspace=ws[1], stream=s2)
            out["fb"] = agk.rmsnorm_fwd(b[0], b[1], 1e-6, workspace=fws[1], stream=s2)
        torch.cuda.synchronize()
        print(f"two streams, round {rep}", flush=True)
        for name, ref in (("fa", ref_fa), ("ba", ref_ba), ("fb", ref_fb), ("bb", ref_bb)):
            assert all(torch.equal(g, r) for g, r in zip(out[name], ref)), (rep, name)


def test_team_is_deterministic(cuda):
    """Three calls of the team kernel on the same inputs: every bit equal."""
    import torch
    x, g, dy = device_inputs((700, 65536), "bf16", 77, cuda)
    _, inv = agk.rmsnorm_fwd(x, g, 1e-6)
    first = agk.rmsnorm_bwd(x, g, inv, dy)
    for _ in range(2):
        again = agk.rmsnorm_bwd(x, g, inv, dy)
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(first, again))


def test_wide_no_gamma(cuda):
    x, _, dy = configs.make_inputs((3, 65536), with_gamma=False, seed=21)
    got = gpu_layer(x, None, dy, 1e-5, cuda)
    _compare(x, None, dy, 1e-5, got, "wide no gamma")


@pytest.mark.parametrize("dtype,rows,cols", [("f32", 5, 40000), ("bf16", 4, 65536),
                                             ("f32", 1, 1 << 20), ("f32", 300, 20480),
                                             ("bf16", 512, 32768)], ids=str)
@pytest.mark.parametrize("flags", [agk.AGK_ACCUM_DX, agk.AGK_ACCUM_DGAMMA, agk.AGK_ACCUM_ALL])
def test_wide_accumulate(cuda, dtype, rows, cols, flags):
    """Each output accumulates on its own (several row blocks through the
    finalize, and one row block whose tiles add into dgamma directly): fp32
    dx and dgamma bit-identical to pre + fresh.  bf16 dx is rounded once from
    pre + the fp32 term, which pre + the bf16-rounded fresh dx cannot
    reproduce bit for bit: within those two roundings (2^-8 relative each)."""
    import torch
    xd, gd, dyd = device_inputs((rows, cols), dtype, rows * 3 + cols + flags, cuda)
    _, inv = agk.rmsnorm_fwd(xd, gd, 1e-6)
    fresh_dx, fresh_dg = agk.rmsnorm_bwd(xd, gd, inv, dyd)
    pre_dx = torch.full_like(xd, 0.25)
    pre_dg = torch.full((cols,), -0.5, device=cuda)
    dx, dg = agk.rmsnorm_bwd(xd, gd, inv, dyd, dx=pre_dx.clone(), dgamma=pre_dg.clone(),
                             accumulate=flags)
    torch.cuda.synchronize()
    want_dg = (pre_dg + fresh_dg) if flags & agk.AGK_ACCUM_DGAMMA else fresh_dg
    assert torch.equal(dg, want_dg)
    if not flags & agk.AGK_ACCUM_DX:
        assert torch.equal(dx, fresh_dx)
    elif dtype == "f32":
        assert torch.equal(dx, pre_dx + fresh_dx)
    else:
        p, f = pre_dx.float(), fresh_dx.float()
        bound = 2.0 ** -7 * (p.abs() + f.abs())
        assert bool(((dx.float() - (p + f)).abs() <= bound).all())


@pytest.mark.parametrize("dtype,rows,cols", [("f32", 6, 65536), ("bf16", 300, 40000),
                                             ("f32", 400, 24576)], ids=str)
def test_wide_one_output(cuda, dtype, rows, cols):
    """dx alone (with a workspace) and dgamma alone: bit-identical to the full
    call's outputs; dx alone without a workspace takes the looped kernel (the
    split path needs the workspace; the one-pass kernel does not, and takes
    it), within the oracle's bar."""
    import torch
    x, g, dy = configs.make_inputs((rows, cols), dtype=dtype, seed=31 + rows)
    xd, gd, dyd = to_dev(x, cuda), to_dev(g, cuda), to_dev(dy, cuda)
    _, inv = agk.rmsnorm_fwd(xd, gd, 1e-6)
    full_dx, full_dg = agk.rmsnorm_bwd(xd, gd, inv, dyd)
    dx_only, none_dg = agk.rmsnorm_bwd(xd, gd, inv, dyd, want_dgamma=False)
    none_dx, dg_only = agk.rmsnorm_bwd(xd, gd, inv, dyd, want_dx=False)
    torch.cuda.synchronize()
    assert none_dg is None and none_dx is None
    assert torch.equal(dx_only, full_dx)
    assert torch.equal(dg_only, full_dg)
    # no workspace: the C ABI with a NULL workspace and dgamma == NULL
    dx_loop = torch.empty_like(xd)
    rc = agk.lib().agk_rmsnorm_bwd(xd.data_ptr(), gd.data_ptr(), inv.data_ptr(), dyd.data_ptr(),
                                   dx_loop.data_ptr(), None, None, 0, rows, cols,
                                   _dt(dtype), 0, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    _, rinv = oracle.fwd(x, g, 1e-6)
    rdx, _ = oracle.bwd(x, g, rinv, dy)
    if _one_pass(rows, cols):
        assert torch.equal(dx_loop, full_dx)
    for name, t in (("with workspace", full_dx), ("without", dx_loop)):
        e = dx_rel_err(as_f32(to_host(t)), as_f32(rdx), as_f32(x), as_f32(g), as_f32(dy), 1e-6)
        print(f"[{dtype} {rows}x{cols} dx {name}] {e:.2e}", flush=True)
        assert e <= _tol(x)


def test_wide_forward_in_place(cuda):
    """y == x: the one-workgroup-per-row kernel (the split forward would
    overwrite x with its partial sums), same bars as out of place."""
    import torch
    rows, cols = 4, 65536
    x, g, dy = configs.make_inputs((rows, cols), seed=41)
    xd, gd = to_dev(x, cuda), to_dev(g, cuda)
    y_out, inv_out = agk.rmsnorm_fwd(xd, gd, 1e-6)
    buf = xd.clone()
    y_in, inv_in = agk.rmsnorm_fwd(buf, gd, 1e-6, y=buf)
    torch.cuda.synchronize()
    assert y_in.data_ptr() == buf.data_ptr()
    ry, rinv = oracle.fwd(x, g, 1e-6)
    for name, y, inv in (("split", y_out, inv_out), ("in place", y_in, inv_in)):
        ey = row_rel_err(to_host(y), ry)
        ei = vec_rel_err(to_host(inv), rinv)
        print(f"[in-place test {name}] y={ey:.2e} inv={ei:.2e}", flush=True)
        assert ey <= TOL_F32 and ei <= TOL_F32


@pytest.mark.parametrize("cols", [40002, 65537])
def test_wide_unaligned_rows(cuda, cols):
    """Rows that are not whole 16-byte slots keep the looped kernels."""
    assert agk.launch_plan(3, cols, agk.AGK_F32, True)["nv"] == 0
    x, g, dy = configs.make_inputs((3, cols), seed=cols)
    got = gpu_layer(x, g, dy, 1e-6, cuda)
    _compare(x, g, dy, 1e-6, got, f"wide unaligned 3x{cols}")


def test_wide_workspace_size(cuda):
    """The workspace query covers the split path's regions, and a call with a
    workspace one byte short of it is refused when dgamma is wanted."""
    import torch
    rows, cols = 300, 65536
    need = agk.rmsnorm_bwd_workspace_bytes(rows, cols)
    assert need >= 16 << 20
    x = torch.randn(rows, cols, device=cuda)
    _, inv = agk.rmsnorm_fwd(x, None, 1e-6)
    ws = torch.empty(need - 1, dtype=torch.uint8, device=cuda)
    with pytest.raises(agk.AgkError) as ei:
        agk.rmsnorm_bwd(x, None, inv, x, workspace=ws)
    assert ei.value.status == 3


@pytest.mark.parametrize("rows,cols", [(6, 65536), (300, 24576)], ids=str)
@pytest.mark.parametrize("fwd_ws", [False, True], ids=["fwd", "fwd_ws"])
def test_wide_paths_under_graph_capture(cuda, rows, cols, fwd_ws):
    """A forward and backward call (the split forward, or with fwd_ws the
    team forward and its slot-clearing fill kernel; the team or the one-pass
    backward, with their partial sums in y and the workspaces) captured once
    into a HIP graph: three replays on new inputs, with eager calls and
    synchronisations between them, each bit-identical to the eager calls on
    the same inputs."""
    import torch
    x = torch.empty(rows, cols, device=cuda)
    dy = torch.empty_like(x)
    g = torch.rand(cols, device=cuda) + 0.5
    y, dx = torch.empty_like(x), torch.empty_like(x)
    inv = torch.empty(rows, device=cuda)
    dg = torch.empty(cols, device=cuda)
    ws = torch.empty(agk.rmsnorm_bwd_workspace_bytes(rows, cols), dtype=torch.uint8, device=cuda)
    fws = False
    if fwd_ws:
        fws = torch.empty(max(agk.rmsnorm_fwd_workspace_bytes(rows, cols), 8), dtype=torch.uint8,
                          device=cuda)
    x.normal_()
    dy.normal_()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = torch.cuda.current_stream()
        agk.rmsnorm_fwd(x, g, 1e-6, y=y, inv_rms=inv, workspace=fws, stream=st)
        agk.rmsnorm_bwd(x, g, inv, dy, dx=dx, dgamma=dg, workspace=ws, stream=st)
    gen = torch.Generator(device=cuda)
    for k in range(3):
        gen.manual_seed(100 + k)
        x.copy_(torch.randn(rows, cols, generator=gen, device=cuda))
        dy.copy_(torch.randn(rows, cols, generator=gen, device=cuda))
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in (y, inv, dx, dg)]
        ey, einv = agk.rmsnorm_fwd(x, g, 1e-6)
        edx, edg = agk.rmsnorm_bwd(x, g, einv, dy)
        torch.cuda.synchronize()
        for name, a, b in zip(("y", "inv_rms", "dx", "dgamma"), got, (ey, einv, edx, edg)):
            assert torch.equal(a, b), (k, name)
    del graph

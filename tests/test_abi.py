"""C ABI of libagk_rmsnorm.so, checked without a GPU.

Loads the library, checks it exports every function include/*.h declares
(and that the ctypes binding covers exactly those), and exercises
the argument validation that runs before any HIP call: null pointers,
negative or overflowing sizes, unknown dtypes, missing or short workspaces.
"""
import ctypes
import os
import re
import subprocess

import pytest

import cgadimpl_amd as agk

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_functions():
    names = set()
    for h in sorted(os.listdir(INCLUDE)):
        if not h.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE, h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(agk_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_expected_entry_points():
    fns = declared_functions()
    for want in ("agk_rmsnorm_fwd", "agk_rmsnorm_fwd_ws", "agk_rmsnorm_bwd",
                 "agk_rmsnorm_bwd_workspace_bytes",
                 "agk_status_str", "agk_rmsnorm_jvp", "agk_layernorm_fwd", "agk_layernorm_bwd",
                 "agk_softmax_fwd", "agk_softmax_bwd", "agk_logsumexp_fwd", "agk_logsumexp_bwd",
                 "agk_logsumexp_jvp", "agk_gemm_bf16"):
        assert want in fns


def test_library_exports_every_declared_symbol():
    path = agk.lib_path()
    assert os.path.exists(path), "build first: python -c 'import __graft_entry__ as g; g.build()'"
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    exported = set(ln.split()[-1] for ln in out.splitlines() if " T " in ln)
    missing = [f for f in declared_functions() if f not in exported]
    assert not missing, missing
    # the ctypes binding covers exactly the header
    assert sorted(agk.SIGNATURES) == declared_functions()
    lib = agk.lib()
    for f in declared_functions():
        assert getattr(lib, f) is not None


def test_status_strings_and_version():
    lib = agk.lib()
    for code, name in agk.STATUS.items():
        assert lib.agk_status_str(code).decode().startswith(name)
    assert b"unknown" in lib.agk_status_str(99)
    assert b"gfx950" in lib.agk_version()


def _blocks(rows):
    rpb = -(-rows // 1024)
    if rows >= 2048:
        rpb = max(rpb, 4)
    return -(-rows // rpb)


def test_workspace_bytes_rule():
    lib = agk.lib()
    ws = lib.agk_rmsnorm_bwd_workspace_bytes
    assert ws(0, 4096) == 0 and ws(16, 0) == 0 and ws(-1, 4) == 0 and ws(4, -1) == 0
    # rows per block = ceil(rows / 1024), at least 4 once rows >= 2048;
    # one fp32 partial row per block
    assert ws(65536, 4096) == 1024 * 4096 * 4
    assert ws(512, 512) == 512 * 512 * 4
    assert ws(51, 13824) == 51 * 13824 * 4
    assert ws(1048576, 128) == 1024 * 128 * 4
    assert ws(7161, 5120) == 1023 * 5120 * 4
    assert ws(2048, 64) == 512 * 64 * 4
    for rows in (1, 2, 255, 256, 257, 1023, 1024, 1025, 2047, 2048, 2049, 4095, 4096, 4097,
                 65535, 10 ** 7):
        assert ws(rows, 8) == _blocks(rows) * 8 * 4, rows
        # resident kernels: 256 workgroups (one partial row each), never more
        # than the workspace holds; below 256 rows, row and column workgroups
        # in one launch and no partial rows
        for dt in (agk.AGK_F32, agk.AGK_BF16):
            plan = agk.launch_plan(rows, 8 * 16, dt, True)
            assert plan["tpr"] > 0
            if rows < 256:
                assert plan["nblk"] == 0 and plan["rpb"] == 0
            else:
                assert plan["nblk"] == 256 <= _blocks(rows)
                assert plan["rpb"] == -(-rows // plan["nblk"])
        # the looped kernel (cols not a whole number of 16-byte slots): runs of
        # rpb consecutive rows, one partial row per run
        plan = agk.launch_plan(rows, 9, agk.AGK_F32, True)
        assert plan["tpr"] == 0 and plan["nblk"] == _blocks(rows)
        assert (plan["nblk"] - 1) * plan["rpb"] < rows <= plan["nblk"] * plan["rpb"]
    assert lib.agk_mul_rowbcast_bwd_workspace_bytes(65536, 4096) == ws(65536, 4096)


def _r256(b):
    return (b + 255) // 256 * 256


def _split_blocks(rows, cols):
    """(row blocks, rows per block) of the split backward: about 2048 tiles of
    2048 columns."""
    nch = -(-cols // 2048)
    nrb = min(max(-(-2048 // nch), 1), rows)
    rb = -(-rows // nrb)
    return -(-rows // rb), rb


def _split_ws(rows, cols, prows):
    """Partial rows, segment slots (8 bytes per 4096 columns), coefficients."""
    return _r256(prows * cols * 4) + _r256(rows * -(-cols // 4096) * 8) + _r256(rows * 4)


def test_wide_row_plans_and_workspace():
    """Rows of AGK_WIDE_MIN_COLS (16385) columns and more: the workspace covers
    the split path's regions (its own row blocks, and the looped blocking the
    composition uses) as well as the looped kernel's partial rows, the same for
    both dtypes; the plan diagnostic reports the one-pass backward from 256
    rows of at most 32768 columns, the team kernel for other aligned rows of
    up to 256 segments from 4 rows, the split paths otherwise (and for every
    wide forward), the looped kernels for rows that are not whole 16-byte
    slots."""
    lib = agk.lib()
    ws = lib.agk_rmsnorm_bwd_workspace_bytes
    assert agk.AGK_WIDE_MIN_COLS == 16385
    for rows in (1, 7, 300, 5000):
        assert ws(rows, 16384) == _blocks(rows) * 16384 * 4  # narrower: unchanged
    for rows, cols in [(1, 1 << 20), (8, 262144), (51, 32768), (255, 32768), (256, 16388),
                       (300, 65536), (4096, 32768), (1100, 20480), (7, 16385), (3, 40002),
                       (1024, 65536), (1023, 65536), (2000, 40004), (12, 131072)]:
        nrb, rb = _split_blocks(rows, cols)
        want = max(_blocks(rows) * cols * 4, _split_ws(rows, cols, nrb),
                   _split_ws(rows, cols, _blocks(rows)))
        assert ws(rows, cols) == want, (rows, cols)
        for dt, w in ((agk.AGK_F32, 4), (agk.AGK_BF16, 8)):
            label = (rows, cols, dt)
            bp = agk.launch_plan(rows, cols, dt, True)
            fp = agk.launch_plan(rows, cols, dt, False)
            if cols % w:
                assert bp["tpr"] == 0 and bp["nv"] == 0, label
                assert fp["tpr"] == 0 and fp["nv"] == 0, label
                continue
            if rows >= 256 and cols <= 32768:
                assert (bp["tpr"], bp["nv"], bp["g"]) == (1024, 32768 // (w * 1024), 1), label
                assert bp["nblk"] == 256 and bp["rpb"] == -(-rows // 256), label
            elif rows >= 4:
                # the team kernel: 8192 bf16 columns per workgroup; fp32 4096,
                # or 8192 where 4096-column parts would be 32 or more or a team
                # of 8192-column parts gets 16 rows or more (given rows for
                # 512 // parts teams); one partial row
                # per team, 512 // parts teams (at most the split path's row
                # blocks)
                part = 8192
                if w == 4:
                    teams2 = max(512 // -(-cols // 8192), 1)
                    if rows < teams2 or (-(-cols // 4096) < 32 and rows < 16 * teams2):
                        part = 4096
                parts = -(-cols // part)
                teams = min(max(512 // parts, 1), nrb)
                assert bp["g"] == 0, label
                assert bp["tpr"] == 256 * parts, label
                assert bp["nv"] == part // (w * 256), label
                assert bp["nblk"] == teams and bp["rpb"] == -(-rows // teams), label
            else:
                assert bp["tpr"] == 0, label
                assert (bp["nv"], bp["g"]) == (-(-cols // 4096), -(-cols // 2048)), label
                assert bp["rpb"] == rb and bp["nblk"] == (nrb if nrb > 1 else 0), label
            if cols // w <= 8192:
                assert fp["tpr"] > 0, label  # the resident forward holds the row
            else:
                assert fp["tpr"] == 0, label
                assert (fp["nv"], fp["g"]) == (-(-cols // 4096), -(-cols // 2048)), label


def _fwd_ws_rule(rows, cols):
    """The documented workspace of agk_rmsnorm_fwd_ws: one 8-byte word per
    row and 4096-column segment for 4+ rows of 16385 to 1M columns, else 0."""
    nseg = -(-cols // 4096)
    return rows * nseg * 8 if cols >= 16385 and nseg <= 256 and rows >= 4 else 0


def test_forward_team_plans_and_workspace():
    """agk_rmsnorm_fwd_ws: its workspace rule, the plan diagnostic's team
    forward (mode 2) wherever agk_rmsnorm_fwd would take the split path
    (16384 bf16 columns per workgroup; fp32 8192, or 16384 where 8192-column
    parts would number 16 or more or a team of them would get at most 4 rows,
    given rows for 512 // parts teams; min(512 // parts, rows) teams), the same plan as agk_rmsnorm_fwd elsewhere
    or with the team switched off, and validation before any HIP call."""
    lib = agk.lib()
    wb = lib.agk_rmsnorm_fwd_workspace_bytes
    for rows, cols in [(8, 262144), (300, 65536), (4, 1 << 20), (7, 50000), (3, 65536),
                       (5, 1 << 21), (600, 40000), (9, 16384), (9, 16385), (0, 65536)]:
        assert wb(rows, cols) == _fwd_ws_rule(rows, cols), (rows, cols)
    assert wb(300, 65536) == 300 * 16 * 8
    for rows, cols in [(8, 262144), (300, 65536), (4, 1 << 20), (7, 50000), (3, 65536),
                       (5, 1 << 21), (600, 40000), (6, 70008), (9, 16388), (5, 40002),
                       (256, 65536), (257, 65536), (2048, 131072), (4096, 40000)]:
        for dt, w in ((agk.AGK_F32, 4), (agk.AGK_BF16, 8)):
            label = (rows, cols, dt)
            plain = agk.launch_plan(rows, cols, dt, False)
            team = agk.launch_plan(rows, cols, dt, False, fwd_workspace=True)
            split = plain["tpr"] == 0 and plain["nv"] > 0
            if split and _fwd_ws_rule(rows, cols):
                part = 16384
                if w == 4:
                    parts2 = -(-cols // 8192)
                    teams4 = max(512 // -(-cols // 16384), 1)
                    if rows < teams4 or (parts2 < 16 and rows > 4 * max(512 // parts2, 1)):
                        part = 8192
                parts = -(-cols // part)
                teams = min(max(512 // parts, 1), rows)
                assert team == {"tpr": 256 * parts, "nv": part // (256 * w), "g": 0,
                                "rpb": -(-rows // teams), "nblk": teams}, label
            else:
                assert team == plain, label
    assert agk.launch_plan(300, 65536, agk.AGK_F32, False, fwd_workspace=True)["g"] == 0
    prev = agk.set_team_forward(0)
    try:
        assert agk.launch_plan(300, 65536, agk.AGK_F32, False, fwd_workspace=True) == \
            agk.launch_plan(300, 65536, agk.AGK_F32, False)
    finally:
        agk.set_team_forward(prev)
    assert agk.set_team_forward(-1) == prev
    assert lib.agk_rmsnorm_launch_plan(8, 65536, 0, 3, (ctypes.c_int32 * 5)()) == 1
    f = lib.agk_rmsnorm_fwd_ws
    need = wb(4, 65536)
    assert f(FAKE, None, FAKE, FAKE, FAKE, need - 1, 4, 65536, 1e-6, 0, None) == 3
    assert f(FAKE, None, FAKE, FAKE, FAKE + 4, need, 4, 65536, 1e-6, 0, None) == 1
    assert f(None, None, FAKE, FAKE, FAKE, need, 4, 65536, 1e-6, 0, None) == 1
    assert f(FAKE, None, FAKE, None, None, 0, 4, 65536, 1e-6, 0, None) == 1
    assert f(FAKE, None, FAKE, FAKE, None, 0, 4, 65536, 1e-6, 9, None) == 2
    assert f(None, None, None, None, None, 0, 0, 65536, 1e-6, 0, None) == 0


def test_launch_plans_are_well_formed():
    """Every reachable resident shape holds its row: lanes * slots * width >= cols."""
    from plans import reachable_plans
    cases = reachable_plans()
    assert len(cases) > 20
    for (dt, direction, tpr, nv, g), reps in cases.items():
        w = 4 if dt == agk.AGK_F32 else 8
        for rows, cols in reps:
            assert tpr * nv * w >= cols
            assert nv == 1 or tpr * nv * w // 2 < cols or tpr == 64, (tpr, nv, cols)
            assert 64 <= tpr * g <= 1024 and (tpr & (tpr - 1)) == 0
            if direction == "bwd":
                assert tpr * g == 1024
    # the headline shapes
    assert agk.launch_plan(65536, 4096, agk.AGK_F32, False)["tpr"] == 512
    bwd = agk.launch_plan(65536, 4096, agk.AGK_F32, True)
    assert (bwd["tpr"], bwd["nv"], bwd["g"], bwd["nblk"]) == (1024, 1, 1, 256)
    # rows that are not whole 16-byte slots take the looped kernels
    assert agk.launch_plan(64, 4098, agk.AGK_F32, False)["tpr"] == 0
    assert agk.launch_plan(64, 4100, agk.AGK_BF16, True)["tpr"] == 0


FAKE = 0x1000  # never dereferenced: validation rejects before any HIP call


def test_fwd_argument_validation():
    lib = agk.lib()
    f = lib.agk_rmsnorm_fwd
    assert f(FAKE, None, FAKE, FAKE, -1, 8, 1e-6, 0, None) == 1
    assert f(FAKE, None, FAKE, FAKE, 8, -1, 1e-6, 0, None) == 1
    assert f(FAKE, None, FAKE, FAKE, 8, 2 ** 31, 1e-6, 0, None) == 1     # cols > INT_MAX
    assert f(FAKE, None, FAKE, FAKE, 2 ** 62, 2 ** 20, 1e-6, 0, None) == 1  # rows*cols overflow
    assert f(FAKE, None, FAKE, FAKE, 8, 8, 1e-6, 7, None) == 2            # dtype
    assert f(None, None, FAKE, FAKE, 8, 8, 1e-6, 0, None) == 1
    assert f(FAKE, None, None, FAKE, 8, 8, 1e-6, 0, None) == 1
    assert f(FAKE, None, FAKE, None, 8, 8, 1e-6, 1, None) == 1
    # empty inputs are a valid no-op, null pointers allowed
    assert f(None, None, None, None, 0, 8, 1e-6, 0, None) == 0
    assert f(None, None, None, None, 8, 0, 1e-6, 0, None) == 0


def test_bwd_argument_validation():
    lib = agk.lib()
    b = lib.agk_rmsnorm_bwd
    args = dict(x=FAKE, g=None, inv=FAKE, dy=FAKE, dx=FAKE, dg=FAKE, ws=FAKE, wsb=1 << 30,
                rows=64, cols=64, dt=0, acc=0)

    def call(**kw):
        a = dict(args, **kw)
        return b(a["x"], a["g"], a["inv"], a["dy"], a["dx"], a["dg"], a["ws"], a["wsb"],
                 a["rows"], a["cols"], a["dt"], a["acc"], None)

    assert call(rows=-2) == 1
    assert call(dt=3) == 2
    assert call(x=None) == 1
    assert call(inv=None) == 1
    assert call(dy=None) == 1
    assert call(acc=4) == 1          # only AGK_ACCUM_DX | AGK_ACCUM_DGAMMA bits exist
    assert call(acc=-1) == 1
    # neither dx nor dgamma requested: a valid no-op (dx alone may be NULL)
    assert call(dx=None, dg=None, ws=None, wsb=0) == 0
    need = lib.agk_rmsnorm_bwd_workspace_bytes(64, 64)
    assert call(ws=None) == 3
    assert call(wsb=need - 1) == 3
    # no dgamma requested: workspace is not needed, but data pointers still are
    assert call(dg=None, ws=None, wsb=0, x=None) == 1
    # empty rows with accumulate: nothing to do
    assert call(rows=0, acc=3, x=None, inv=None, dy=None, dx=None, ws=None, wsb=0) == 0


def test_mul_argument_validation():
    lib = agk.lib()
    assert lib.agk_mul_rowbcast_fwd(None, FAKE, FAKE, 4, 4, 0, None) == 1
    assert lib.agk_mul_rowbcast_fwd(FAKE, FAKE, FAKE, 4, 4, 5, None) == 2
    assert lib.agk_mul_rowbcast_fwd(None, None, None, 0, 4, 0, None) == 0
    m = lib.agk_mul_rowbcast_bwd
    assert m(None, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 20, 4, 4, 0, 0, None) == 1  # gy
    assert m(FAKE, FAKE, None, FAKE, None, None, 0, 4, 4, 0, 0, None) == 1        # da needs b
    assert m(FAKE, None, FAKE, None, FAKE, FAKE, 1 << 20, 4, 4, 0, 0, None) == 1  # db needs a
    assert m(FAKE, FAKE, FAKE, None, FAKE, None, 0, 4, 4, 0, 0, None) == 3        # db needs ws
    assert m(FAKE, FAKE, FAKE, None, None, None, 0, 4, 4, 0, 0, None) == 0        # nothing asked
    assert m(FAKE, FAKE, FAKE, FAKE, None, None, 0, 4, 4, 0, 8, None) == 1        # bad accumulate
    sr = lib.agk_sum_rows  # x, out, ws, wsb, rows, cols, dtype, accumulate
    assert sr(None, FAKE, FAKE, 1 << 20, 4, 4, 0, 0, None) == 1                # x
    assert sr(FAKE, None, FAKE, 1 << 20, 4, 4, 0, 0, None) == 1                # out
    assert sr(FAKE, FAKE, None, 0, 4, 4, 0, 0, None) == 3                      # workspace
    assert sr(FAKE, FAKE, FAKE, 1 << 20, 4, 4, 3, 0, None) == 2                # dtype
    assert sr(FAKE, FAKE, FAKE, 1 << 20, 4, 4, 0, 2, None) == 1                # accumulate
    assert sr(None, None, None, 0, 4, 0, 0, 0, None) == 0                      # no columns
    assert lib.agk_sum_rows_workspace_bytes(65536, 4096) == lib.agk_rmsnorm_bwd_workspace_bytes(65536, 4096)
    li = lib.agk_linear_bf16  # X, ldx, W, ldw, bias, Y, ldy, M, N, K
    assert li(None, 64, FAKE, 64, FAKE, FAKE, 64, 64, 64, 64, None) == 1     # X
    assert li(FAKE, 64, FAKE, 64, FAKE + 1, FAKE, 64, 64, 64, 64, None) == 1  # odd bias
    assert li(FAKE, 60, FAKE, 64, None, FAKE, 64, 64, 64, 64, None) == 1     # ldx
    assert li(FAKE, 64, FAKE, 64, None, FAKE, 32, 64, 64, 64, None) == 1     # ldy < N
    assert li(None, 0, None, 0, None, None, 0, 0, 64, 64, None) == 0         # no rows
    r = lib.agk_rms_mul_bwd  # x, gamma, inv, gy, dr, dx, dgamma, ws, wsb, rows, cols, dt, acc
    for i in range(5):  # x, gamma, inv_rms, gy and dr are required
        args = [FAKE] * 5
        args[i] = None
        assert r(*args, FAKE, None, None, 0, 4, 4, 0, 0, None) == 1
    assert r(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, 0, 4, 4, 0, 0, None) == 3  # ws
    assert r(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, None, 0, 4, 4, 7, 0, None) == 2  # dtype
    assert r(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, None, 0, 4, 4, 0, 4, None) == 1  # acc bits
    assert r(None, None, None, None, None, None, None, None, 0, 0, 4, 0, 2, None) == 0  # empty


def _shape(*dims):
    return (ctypes.c_int64 * max(1, len(dims)))(*dims), len(dims)


def test_broadcast_shape_rule():
    """agk_mul_bcast_shape follows numpy's rules (compared with numpy itself)."""
    import numpy as np
    lib = agk.lib()
    pairs = [((3, 4), (4,)), ((2, 3, 4), (3, 1)), ((1,), (5, 6)), ((), (2,)), ((), ()),
             ((2, 1, 3, 1), (1, 4, 1, 5)), ((0, 4), (1, 4)), ((7,), (1, 7)), ((3, 4), (2, 4)),
             ((3,), (4,)), ((2, 0), (2, 3))]
    for sa, sb in pairs:
        a, an = _shape(*sa)
        b, bn = _shape(*sb)
        out = (ctypes.c_int64 * 8)()
        nd = ctypes.c_int(-1)
        rc = lib.agk_mul_bcast_shape(a, an, b, bn, out, ctypes.byref(nd))
        try:
            want = np.broadcast_shapes(sa, sb)
        except ValueError:
            assert rc == 1, (sa, sb)
            continue
        assert rc == 0 and tuple(out[i] for i in range(nd.value)) == want, (sa, sb)
    nine, n9 = _shape(*([1] * 9))
    one, n1 = _shape(1)
    nd = ctypes.c_int(0)
    assert lib.agk_mul_bcast_shape(nine, n9, one, n1, None, ctypes.byref(nd)) == 1  # > 8 axes
    neg, nn = _shape(-1, 4)
    assert lib.agk_mul_bcast_shape(neg, nn, one, n1, None, ctypes.byref(nd)) == 1   # negative
    assert lib.agk_mul_bcast_shape(one, n1, one, n1, None, None) == 1               # no out_ndim


def test_broadcast_mul_argument_validation():
    lib = agk.lib()
    a, an = _shape(3, 4)
    b, bn = _shape(4)
    bad, badn = _shape(2, 4)
    e, en = _shape(0, 4)
    f = lib.agk_mul_bcast_fwd  # a, a_shape, a_ndim, b, b_shape, b_ndim, y, dtype, acc
    assert f(FAKE, a, an, FAKE, bad, badn, FAKE, 0, 0, None) == 1    # shapes do not broadcast
    assert f(FAKE, a, an, FAKE, b, bn, FAKE, 3, 0, None) == 2        # dtype
    assert f(None, a, an, FAKE, b, bn, FAKE, 0, 0, None) == 1        # a
    assert f(FAKE, a, an, FAKE, b, bn, None, 0, 0, None) == 1        # y
    assert f(None, e, en, None, b, bn, None, 0, 0, None) == 0        # empty output
    g = lib.agk_mul_bcast_bwd  # gy, a, a_shape, a_ndim, b, b_shape, b_ndim, da, db, dt, acc
    assert g(FAKE, FAKE, a, an, FAKE, bad, badn, FAKE, FAKE, 0, 0, None) == 1  # shapes
    assert g(FAKE, FAKE, a, an, FAKE, b, bn, FAKE, FAKE, 5, 0, None) == 2      # dtype
    assert g(FAKE, FAKE, a, an, FAKE, b, bn, FAKE, FAKE, 0, 4, None) == 1      # accumulate bits
    assert g(None, FAKE, a, an, FAKE, b, bn, FAKE, None, 0, 0, None) == 1      # gy
    assert g(FAKE, FAKE, a, an, None, b, bn, FAKE, None, 0, 0, None) == 1      # da needs b
    assert g(FAKE, None, a, an, FAKE, b, bn, None, FAKE, 0, 0, None) == 1      # db needs a
    assert g(FAKE, FAKE, a, an, FAKE, b, bn, None, None, 0, 0, None) == 0      # nothing asked
    assert g(None, None, e, en, None, b, bn, None, FAKE, 0, 3, None) == 0      # empty, accumulate


def test_gemm_f32_argument_validation():
    lib = agk.lib()
    g = lib.agk_gemm_f32  # A, lda, a_trans, B, ldb, b_trans, C, ldc, M, N, K, accumulate
    assert g(FAKE, 8, 0, FAKE, 8, 0, FAKE, 8, -1, 8, 8, 0, None) == 1          # negative M
    assert g(FAKE, 8, 0, FAKE, 8, 0, FAKE, 8, 8, 8, 1 << 31, 0, None) == 1     # K past int32
    assert g(None, 8, 0, None, 8, 0, None, 8, 0, 8, 8, 0, None) == 0           # no rows
    assert g(FAKE, 8, 0, FAKE, 8, 0, None, 8, 8, 8, 8, 0, None) == 1           # C
    assert g(FAKE, 8, 0, FAKE, 8, 0, FAKE, 7, 8, 8, 8, 0, None) == 1           # ldc < N
    assert g(None, 8, 0, FAKE, 8, 0, FAKE, 8, 8, 8, 8, 0, None) == 1           # A with K > 0
    assert g(FAKE, 7, 0, FAKE, 8, 0, FAKE, 8, 8, 8, 8, 0, None) == 1           # lda < K
    assert g(FAKE, 7, 1, FAKE, 8, 0, FAKE, 8, 8, 8, 8, 0, None) == 1           # lda < M (A^T)
    assert g(FAKE, 8, 0, FAKE, 7, 0, FAKE, 8, 8, 8, 8, 0, None) == 1           # ldb < N
    assert g(FAKE, 8, 0, FAKE, 7, 1, FAKE, 8, 8, 8, 8, 0, None) == 1           # ldb < K (B^T)


def test_rowops_argument_validation():
    lib = agk.lib()
    j = lib.agk_rmsnorm_jvp
    assert j(None, None, FAKE, FAKE, None, FAKE, 4, 8, 0, None) == 1           # x
    assert j(FAKE, None, None, FAKE, None, FAKE, 4, 8, 0, None) == 1           # inv_rms
    assert j(FAKE, None, FAKE, None, None, FAKE, 4, 8, 0, None) == 1           # tx
    assert j(FAKE, None, FAKE, FAKE, None, None, 4, 8, 0, None) == 1           # ty
    assert j(FAKE, None, FAKE, FAKE, FAKE, FAKE, 4, 8, 0, None) == 1           # tgamma w/o gamma
    assert j(FAKE, FAKE, FAKE, FAKE, None, FAKE, 4, 8, 9, None) == 2           # dtype
    assert j(None, None, None, None, None, None, 0, 8, 0, None) == 0           # empty
    assert j(FAKE, FAKE, FAKE, FAKE, None, FAKE, -4, 8, 0, None) == 1          # size

    lf = lib.agk_layernorm_fwd
    assert lf(None, FAKE, FAKE, FAKE, 4, 8, 1e-5, 0, None) == 1
    assert lf(FAKE, FAKE, None, FAKE, 4, 8, 1e-5, 0, None) == 1
    assert lf(FAKE, FAKE, FAKE, None, 4, 8, 1e-5, 0, None) == 1
    assert lf(FAKE, FAKE, FAKE, FAKE, 4, 8, 1e-5, 2, None) == 2
    assert lf(None, None, None, None, 4, 0, 1e-5, 0, None) == 0
    lb = lib.agk_layernorm_bwd
    assert lb(FAKE, FAKE, FAKE, FAKE, None, 4, 8, 0, 0, None) == 1             # dx
    assert lb(FAKE, None, FAKE, FAKE, FAKE, 4, 8, 0, 0, None) == 1             # mean
    assert lb(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 8, 0, 2, None) == 1             # no dgamma here
    assert lb(None, None, None, None, None, 0, 8, 0, 1, None) == 0

    assert lib.agk_softmax_fwd(None, FAKE, 4, 8, 0, None) == 1
    assert lib.agk_softmax_fwd(FAKE, FAKE, 4, 8, 3, None) == 2
    assert lib.agk_softmax_fwd(None, None, 0, 8, 0, None) == 0
    sb = lib.agk_softmax_bwd
    assert sb(FAKE, None, FAKE, 4, 8, 0, 0, None) == 1
    assert sb(FAKE, FAKE, FAKE, 4, 8, 0, 3, None) == 1
    assert sb(None, None, None, 4, 0, 0, 1, None) == 0

    assert lib.agk_logsumexp_fwd(FAKE, FAKE, 4, 0, 0, None) == 1   # log-sum-exp of empty rows
    assert lib.agk_logsumexp_fwd(None, None, 0, 0, 0, None) == 0
    assert lib.agk_logsumexp_fwd(FAKE, None, 4, 8, 0, None) == 1
    assert lib.agk_logsumexp_bwd(FAKE, None, FAKE, 4, 8, 0, 0, None) == 1
    assert lib.agk_logsumexp_bwd(FAKE, FAKE, FAKE, 4, 8, 0, -1, None) == 1
    assert lib.agk_logsumexp_jvp(FAKE, FAKE, FAKE, 4, 0, 0, None) == 1
    assert lib.agk_logsumexp_jvp(FAKE, None, FAKE, 4, 8, 0, None) == 1
    assert lib.agk_logsumexp_jvp(FAKE, FAKE, FAKE, 4, 8, 1 << 20, None) == 2


def _rowops_ws_rule(rows, cols):
    """The documented workspace of the *_ws row ops: two 8-byte values per
    part and row, parts = ceil(ceil(cols / W) / 2048), the most over W = 4
    (fp32) and 8 (bf16) with 2-64 parts."""
    most = 0
    for w in (4, 8):
        parts = -(-(-(-cols // w)) // 2048)
        if 2 <= parts <= 64:
            most = max(most, rows * parts * 16)
    return most


def test_rowops_workspace_rule_and_team_plans():
    """The *_ws row ops' workspace (the most any op uses at the shape, 0 for
    rows one workgroup holds), the team plans in the default mode (aligned
    rows from 3 parts of 2048 16-byte slots, 4 for the softmax backward; rows
    off a boundary from 4 parts, 2 for the softmax backward), and validation
    that rejects a workspace before any HIP call."""
    lib = agk.lib()
    wb = lib.agk_rowops_workspace_bytes
    for rows, cols in [(8192, 128256), (3, 50257), (1, 8193), (5, 262144), (2, 1 << 19),
                       (7, 1 << 20), (9, 6200)]:
        assert wb(rows, cols) == _rowops_ws_rule(rows, cols), (rows, cols)
    assert wb(8192, 128256) == 8192 * 16 * 2 * 8        # fp32 forward: 16 parts, 2 values
    assert wb(100, 4096) == 0 and wb(4, 512) == 0 and wb(0, 131072) == 0
    assert wb(4, 1 << 22) == 0  # more than 64 parts: the team kernel holds no such row
    plan = agk.rowops_team_plan
    # bf16 Llama 3 vocabulary: 16032 slots -> 8 parts of 2004; grid / 8 teams, the
    # grid 3 workgroups per CU of 256 for the two-value ops, 2 for the softmax backward
    for op in agk.ROWOPS_TEAM_OPS:
        assert plan(op, 8192, 128256, 1, True) == {
            "parts": 8, "slots_per_part": 2004, "teams": 64 if op == "softmax_bwd" else 96}
    assert plan("softmax_fwd", 8192, 128256, 0, True)["parts"] == 16
    # aligned rows: the forward and the log-sum-exp backward from 3 parts, the
    # softmax backward from 4 (below, the resident kernels)
    assert plan("softmax_fwd", 4, 65536, 1, True)["parts"] == 4   # bf16 8192 slots
    assert plan("logsumexp_bwd", 4, 40000, 1, True)["parts"] == 3
    assert plan("softmax_fwd", 4, 32000, 1, True)["parts"] == 0   # 2 parts
    assert plan("softmax_fwd", 4, 65536, 0, True)["parts"] == 8
    assert plan("softmax_bwd", 4, 65536, 1, True)["parts"] == 4
    assert plan("softmax_bwd", 4, 40000, 1, True)["parts"] == 0   # 3 parts
    # rows off a 16-byte boundary: the backward from 2 parts, the others from 4
    assert plan("softmax_bwd", 9, 50257, 1, False) == {"parts": 4, "slots_per_part": 1571,
                                                       "teams": 9}
    assert plan("softmax_fwd", 9000, 50257, 1, False) == {"parts": 4, "slots_per_part": 1571,
                                                          "teams": 192}
    assert plan("logsumexp_bwd", 9, 40004, 1, False)["parts"] == 0  # 3 parts
    assert plan("logsumexp_bwd", 9, 50257, 0, False)["parts"] == 7
    assert plan("softmax_fwd", 3, 16384, 1, False)["parts"] == 0  # 2048 slots: one workgroup
    prev = agk.set_rowops_team(0)
    try:
        assert plan("softmax_fwd", 8192, 128256, 1, True)["parts"] == 0
        assert agk.set_rowops_team(2) == 0
        assert plan("softmax_fwd", 3, 16384, 1, False)["parts"] == 1
    finally:
        agk.set_rowops_team(prev)
    assert agk.set_rowops_team(-1) == prev
    assert lib.agk_rowops_team_plan(3, 4, 8, 0, 1, (ctypes.c_int32 * 3)()) == 1
    need = wb(4, 131072)
    assert lib.agk_softmax_fwd_ws(FAKE, FAKE, FAKE, need - 1, 4, 131072, 1, None) == 3
    assert lib.agk_softmax_fwd_ws(FAKE, FAKE, FAKE + 4, need, 4, 131072, 1, None) == 1
    assert lib.agk_softmax_bwd_ws(FAKE, FAKE, FAKE, FAKE, need - 8, 4, 131072, 1, 0, None) == 3
    assert lib.agk_softmax_bwd_ws(FAKE, None, FAKE, None, 0, 4, 131072, 1, 0, None) == 1
    assert lib.agk_softmax_bwd_ws(FAKE, FAKE, FAKE, None, 0, 4, 131072, 1, 2, None) == 1
    assert lib.agk_logsumexp_bwd_ws(FAKE, FAKE, FAKE, FAKE, 0, 4, 131072, 0, 0, None) == 3
    assert lib.agk_logsumexp_bwd_ws(None, FAKE, FAKE, None, 0, 4, 8, 0, 0, None) == 1
    assert lib.agk_softmax_fwd_ws(None, None, None, 0, 0, 8, 0, None) == 0
    assert lib.agk_softmax_fwd_ws(FAKE, FAKE, None, 0, 4, 8, 5, None) == 2


def test_python_binding_raises_without_gpu_tensors():
    torch = pytest.importorskip("torch")
    x = torch.zeros(4, 8)
    with pytest.raises(ValueError):
        agk.rmsnorm_fwd(x, None, 1e-6, y=x, inv_rms=torch.zeros(4))


def test_linear_bf16_rejects_bad_bias_and_output():
    """Checked before any device call: an fp32 bias would be read as pairs of
    bf16 values, a short bias or a mis-shaped y would be read or written out
    of bounds by the kernel."""
    import torch
    x = torch.zeros(16, 32, dtype=torch.bfloat16)
    w = torch.zeros(8, 32, dtype=torch.bfloat16)
    with pytest.raises(TypeError):
        agk.linear_bf16(x, w, torch.zeros(8, dtype=torch.float32))
    with pytest.raises(ValueError):
        agk.linear_bf16(x, w, torch.zeros(4, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        agk.linear_bf16(x, w, torch.zeros(16, dtype=torch.bfloat16)[::2])
    with pytest.raises(ValueError):
        agk.linear_bf16(x, w, None, y=torch.zeros(16, 4, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        agk.linear_bf16(x, w, None, y=torch.zeros(16, 8, dtype=torch.float32))


def test_sanitized_builds_are_the_ones_loaded():
    """Under tests/run_sanitized.py (ORACLE_SANITIZE=1): the libraries the bindings
    load are the sanitised builds, whose host code calls the AddressSanitizer
    runtime.  Skipped in an ordinary run."""
    if os.environ.get("ORACLE_SANITIZE") != "1":
        pytest.skip("not a sanitised run")
    import oracle
    paths = [agk.lib_path(), os.path.join(agk.LIB_DIR, "libagk_synth.so"),
             os.path.join(agk.LIB_DIR, "libag.so"), oracle.build.lib_path()]
    assert agk.lib_path().startswith(os.environ["AGK_LIB_DIR"])
    assert oracle.build.lib_path().startswith(os.environ["ORACLE_LIB_DIR"])
    for p in paths:
        syms = subprocess.run(["nm", "-D", p], capture_output=True, text=True, check=True).stdout
        assert "__asan_" in syms and "__ubsan_" in syms, p
    agk.lib()
    oracle.load()

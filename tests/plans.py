"""Launch shapes the library can pick, with representative sizes for each.

The shape of a call depends on the row width (in 16-byte slots) and on
whether the row count is above the library's large-batch threshold (16384
rows), so every reachable shape is found by walking the widths at one small
and one large row count.  Each shape keeps the narrowest and the widest width
that maps to it (most idle lanes, fully packed lanes).
"""
from __future__ import annotations

import functools

import cgadimpl_amd as agk

SMALL_ROWS = 37        # ragged against every rows-per-workgroup value
LARGE_ROWS = 16411     # above the large-batch threshold, ragged
MAX_SLOTS = 8192       # widest resident forward: 1024 lanes x 8 slots


@functools.lru_cache(maxsize=None)
def reachable_plans():
    """{(dtype, "fwd"|"bwd", tpr, nv, g): [(rows, cols), ...]} for resident shapes."""
    span = {}
    for dt, w in ((agk.AGK_F32, 4), (agk.AGK_BF16, 8)):
        for rows in (SMALL_ROWS, LARGE_ROWS):
            for direction in ("fwd", "bwd"):
                for nslot in range(1, MAX_SLOTS + 1):
                    p = agk.launch_plan(rows, nslot * w, dt, direction == "bwd")
                    if p["tpr"] == 0 or p["g"] == 0:  # not resident: looped, split or team
                        continue
                    key = (dt, direction, p["tpr"], p["nv"], p["g"])
                    lo, hi = span.get((key, rows), (nslot * w, nslot * w))
                    span[(key, rows)] = (min(lo, nslot * w), max(hi, nslot * w))
    out = {}
    for (key, rows), (lo, hi) in span.items():
        out.setdefault(key, set()).update({(rows, lo), (rows, hi)})
    return {k: sorted(v) for k, v in out.items()}

"""Summaries of rocprofv3 output for the RMSNorm kernels (maintainer tool).

Turns the CSV files of two kinds of rocprofv3 runs into short text summaries
under profiles/:

  kernel trace   rocprofv3 --kernel-trace --stats -T -d <dir> -o run -f csv -- <cmd>
                 -> per-kernel calls and average / min / max duration
  HBM traffic    rocprofv3 --pmc FETCH_SIZE ... and --pmc WRITE_SIZE ..., for the
                 workload and for `bench.py --copy-probe MIB` (a device copy of
                 known size), -> HBM bytes per dispatch of each kernel

FETCH_SIZE and WRITE_SIZE are reported in KiB per dispatch.  Each counter is
scaled by what it reads for the copy kernel, whose true traffic is MIB MiB
read and MIB MiB written, so the scaled figures are bytes that actually
crossed the HBM interface.

  MFMA use       rocprofv3 --pmc SQ_INSTS_VALU_MFMA_MOPS_BF16 SQ_VALU_MFMA_BUSY_CYCLES ...
                 -> per GEMM launch shape: flops (512 per MOPS_BF16 count), TFLOP/s,
                 and MFMA-busy time (SQ_VALU_MFMA_BUSY_CYCLES summed over the 1024
                 SIMDs, at the 2.4 GHz peak engine clock) as a share of the kernel time

Usage:
  python -m cgadimpl_amd.profiling trace  <run_kernel_stats.csv> <out.md> "<command>"
  python -m cgadimpl_amd.profiling mfma <run_counter_collection.csv> <out.md> "<command>"
  python -m cgadimpl_amd.profiling bench <bench output (JSON lines)> <out.md> "<command>"
  python -m cgadimpl_amd.profiling probe <bench --stream-probe output> <out.md> "<command>"
  python -m cgadimpl_amd.profiling mfma-probe <bench --mfma-probe output> <out.md> "<command>"
  python -m cgadimpl_amd.profiling gemm-f32 <bench --gemm-f32 output> <out.md> "<command>"
  python -m cgadimpl_amd.profiling wide <bench --wide output> <out.md> "<command>"
  python -m cgadimpl_amd.profiling traffic <fetch_dir> <write_dir> <copy_fetch_dir>
        <copy_write_dir> <copy_mib> <config> <out_stem> "<command>"
  python -m cgadimpl_amd.profiling gemm-traffic <fetch_dir> <write_dir> <copy_fetch_dir>
        <copy_write_dir> <copy_mib> <out.md> "<command>"
  python -m cgadimpl_amd.profiling wide-traffic <out.md> "<command>" <copy_mib>
        <copy_fetch_dir> <copy_write_dir> <label>,<fetch_dir>,<write_dir>,<bench output> ...
"""
from __future__ import annotations

import csv
import json
import os
import sys
from collections import defaultdict

# Kernels that make up one call of each C-ABI entry point.
# entry point: (its main kernels, kernels a call adds after one of them)
ENTRY_KERNELS = {
    "agk_rmsnorm_fwd": (("rms_fwd_resident", "rms_fwd_looped"), ()),
    "agk_rmsnorm_bwd": (("rms_bwd_resident", "rms_bwd_looped", "bwd_fewrows"),
                        ("dgamma_finalize", "dgamma_finalize_few")),
    "agk_rms_mul_bwd": (("rms_mul_bwd_resident",), ("dgamma_finalize", "dgamma_finalize_few")),
}

# The files the RMSNorm kernels are compiled from.  A traffic summary records a
# hash of them, and bench.py uses a summary only while the hash still matches.
KERNEL_SOURCES = ("cgadimpl_amd/csrc/rmsnorm.hip", "cgadimpl_amd/csrc/rowcommon.hpp",
                  "cgadimpl_amd/csrc/rmsnorm_wide.hpp")


def kernel_source_hash(root=None):
    """sha256 over the RMSNorm kernel sources (KERNEL_SOURCES, in order)."""
    import hashlib
    root = root or os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        with open(os.path.join(root, rel), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()


def _git_head(root):
    import subprocess
    try:
        return subprocess.run(["git", "-C", root, "rev-parse", "--short=12", "HEAD"],
                              capture_output=True, text=True, check=True).stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        return None


def _rows(path):
    with open(path, newline="") as fh:
        return list(csv.DictReader(fh))


def kernel_stats(stats_csv):
    """{kernel: (calls, avg_ns, min_ns, max_ns)} from run_kernel_stats.csv."""
    out = {}
    for r in _rows(stats_csv):
        out[r["Name"]] = (int(r["Calls"]), float(r["AverageNs"]), float(r["MinNs"]),
                          float(r["MaxNs"]))
    return out


def short_name(name):
    """Kernel names shortened for the tables: hipBLASLt's long tuned names, and full
    (untruncated) device names cut to the kernel and its template arguments without
    namespaces, e.g. "row_resident<BF16, 512, 2, 1, LseFwd>"."""
    if name.startswith(("Cijk_", "Custom_Cijk_")):
        return "hipBLASLt " + name.split("_MT")[0] + ("_MT" + name.split("_MT")[1][:12]
                                                      if "_MT" in name else "")
    if name.startswith("void "):
        name = name[len("void "):]
    depth = 0
    for i, ch in enumerate(name):  # drop the parameter list: the first '(' outside <...>
        depth += ch == "<"
        depth -= ch == ">"
        if ch == "(" and depth == 0:
            name = name[:i]
            break
    for ns in ("agk::rowops::", "agk_gemm::", "agk::", "at::native::"):
        name = name.replace(ns, "")
    if not name:
        return "(torch, unnamed)"
    if name.startswith(("vectorized_elementwise_kernel", "elementwise_kernel",
                        "distribution_elementwise", "index_elementwise", "reduce_kernel")):
        return "torch " + name.split("<")[0]  # input generation, not this build's kernels
    return name


def dispatch_stats(trace_csv):
    """{(kernel, grid, workgroup): [durations ns]} from run_kernel_trace.csv."""
    out = defaultdict(list)
    for r in _rows(trace_csv):
        key = (r["Kernel_Name"], f'{r["Grid_Size_X"]}x{r["Grid_Size_Y"]}',
               r["Workgroup_Size_X"])
        out[key].append(float(r["End_Timestamp"]) - float(r["Start_Timestamp"]))
    return out


def write_trace_summary(stats_csv, out_md, command):
    st = kernel_stats(stats_csv)
    lines = ["# Kernel durations (rocprofv3 --kernel-trace --stats)", "",
             "Command:", "", "```", command, "```", "",
             "| kernel | calls | avg us | min us | max us |", "|---|---|---|---|---|"]
    for name, (calls, avg, mn, mx) in sorted(st.items(), key=lambda kv: -kv[1][0] * kv[1][1]):
        lines.append(f"| {short_name(name)} | {calls} | {avg / 1e3:.1f} | {mn / 1e3:.1f} | "
                     f"{mx / 1e3:.1f} |")
    lines.append("")
    trace_csv = os.path.join(os.path.dirname(stats_csv),
                             os.path.basename(stats_csv).replace("kernel_stats", "kernel_trace"))
    if os.path.exists(trace_csv):
        lines += ["Per launch shape (grid threads x, y; workgroup size), from the trace:", "",
                  "| kernel | grid | workgroup | calls | avg us |", "|---|---|---|---|---|"]
        ds = dispatch_stats(trace_csv)
        for (name, grid, wg), v in sorted(ds.items(), key=lambda kv: -sum(kv[1])):
            lines.append(f"| {short_name(name)} | {grid} | {wg} | {len(v)} | "
                         f"{sum(v) / len(v) / 1e3:.1f} |")
        lines.append("")
    for entry, (main, extra) in ENTRY_KERNELS.items():
        if not any(k in st for k in main):
            continue
        kernels = [k for k in main + extra if k in st]
        tot = sum(st[k][1] for k in kernels)
        lines.append(f"- one `{entry}` call: {tot / 1e3:.1f} us ({' + '.join(kernels)})")
    with open(out_md, "w") as fh:
        fh.write("\n".join(lines) + "\n")


def _counter_by_kernel(run_dir, counter):
    """{kernel: [per-dispatch values]} of one counter (KiB per dispatch)."""
    vals = defaultdict(list)
    for r in _rows(os.path.join(run_dir, "run_counter_collection.csv")):
        if r["Counter_Name"] == counter:
            vals[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return vals


def _median(v):
    s = sorted(v)
    return s[len(s) // 2]


def traffic(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir, copy_mib):
    """Scaled HBM bytes per dispatch: {kernel: (read_bytes, write_bytes)}, factors."""
    cf = _counter_by_kernel(copy_fetch_dir, "FETCH_SIZE")
    cw = _counter_by_kernel(copy_write_dir, "WRITE_SIZE")
    copy_kib = copy_mib * 1024.0
    fetch_scale = copy_kib / _median(next(v for k, v in cf.items() if "copy" in k.lower()))
    write_scale = copy_kib / _median(next(v for k, v in cw.items() if "copy" in k.lower()))
    f = _counter_by_kernel(fetch_dir, "FETCH_SIZE")
    w = _counter_by_kernel(write_dir, "WRITE_SIZE")
    out = {}
    for k in set(f) | set(w):
        rd = _median(f[k]) * fetch_scale * 1024.0 if k in f else 0.0
        wr = _median(w[k]) * write_scale * 1024.0 if k in w else 0.0
        out[k] = (rd, wr)
    return out, fetch_scale, write_scale


def write_traffic_summary(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir, copy_mib,
                          config, out_stem, command):
    from . import configs
    cfg = configs.CONFIGS[config]
    per_kernel, fs, ws = traffic(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir,
                                 copy_mib)
    alg = {"agk_rmsnorm_fwd": cfg.fwd_bytes(), "agk_rmsnorm_bwd": cfg.bwd_bytes()}
    lines = [f"# HBM traffic per call, configuration {config} {list(cfg.shape)} {cfg.dtype}",
             "", "Commands (each counter in its own run):", "", "```", command, "```", "",
             f"Counter scale from a {copy_mib} MiB device copy (`bench.py --copy-probe "
             f"{copy_mib}`): FETCH_SIZE x {fs:.4f}, WRITE_SIZE x {ws:.4f}.", "",
             "| kernel | read MB | write MB |", "|---|---|---|"]
    layer = {e: ENTRY_KERNELS[e][0] + ENTRY_KERNELS[e][1] for e in alg}
    for k, (rd, wr) in sorted(per_kernel.items()):
        if any(k in ks for ks in layer.values()):
            lines.append(f"| {k} | {rd / 1e6:.1f} | {wr / 1e6:.1f} |")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    src = kernel_source_hash(root)
    rec = {"config": config, "fetch_scale": fs, "write_scale": ws,
           "kernel_source_sha256": src, "git_head": _git_head(root)}
    lines += ["", "| entry point | HBM bytes | algorithmic bytes | ratio |", "|---|---|---|---|"]
    for entry, kernels in layer.items():
        tot = sum(sum(per_kernel[k]) for k in kernels if k in per_kernel)
        lines.append(f"| {entry} | {tot:.4g} | {alg[entry]:.4g} | {tot / alg[entry]:.4f} |")
        rec[entry.replace("agk_rmsnorm_", "") + "_hbm_bytes_per_launch"] = round(tot)
    lines += ["", f"Kernel sources ({', '.join(KERNEL_SOURCES)}) sha256 {src[:16]}; git HEAD "
              f"{rec['git_head']} when summarised (uncommitted changes are in the hash)."]
    with open(out_stem + ".md", "w") as fh:
        fh.write("\n".join(lines) + "\n")
    with open(out_stem + ".json", "w") as fh:
        json.dump(rec, fh, indent=1)
        fh.write("\n")


# Kernel-name prefixes of the RMSNorm library's kernels (the rest of a run's
# dispatches are torch's input generation).
LIB_KERNEL_PREFIXES = ("fill_zero_f32", "wide_", "dgamma_finalize", "rms_", "bwd_fewrows",
                       "row_", "team_clear", "lse_bwd_from_value")


def write_wide_traffic_summary(out_md, command, copy_mib, copy_fetch_dir, copy_write_dir,
                               runs):
    """HBM bytes per wide-row call (bench.py --wide-call runs): each run's
    library kernels (medians per kernel over the run's dispatches, scaled by the
    copy's counters) summed against the call's algorithmic bytes.  runs:
    [(label, fetch_dir, write_dir, jsonl_with_the_call_line)]."""
    cf = _counter_by_kernel(copy_fetch_dir, "FETCH_SIZE")
    cw = _counter_by_kernel(copy_write_dir, "WRITE_SIZE")
    copy_kib = copy_mib * 1024.0
    fs = copy_kib / _median(next(v for k, v in cf.items() if "copy" in k.lower()))
    wsc = copy_kib / _median(next(v for k, v in cw.items() if "copy" in k.lower()))
    lines = ["# HBM traffic of wide-row calls: team kernels against the paths without them",
             "", "Commands (each counter in its own run):", "", "```", command, "```", "",
             f"Counter scale from a {copy_mib} MiB device copy (`bench.py --copy-probe "
             f"{copy_mib}`): FETCH_SIZE x {fs:.4f}, WRITE_SIZE x {wsc:.4f}. Each run makes "
             "its inputs with torch and repeats one call three times; the library's kernels "
             "are medians over their dispatches, summed per call.", "",
             "| call | kernels | read MB | write MB | HBM bytes | algorithmic bytes | ratio |",
             "|---|---|---|---|---|---|---|"]
    for label, fdir, wdir, jsonl in runs:
        rec = next(json.loads(ln) for ln in open(jsonl) if ln.startswith('{"wide_call"'))
        f = _counter_by_kernel(fdir, "FETCH_SIZE")
        w = _counter_by_kernel(wdir, "WRITE_SIZE")
        names = sorted(k for k in set(f) | set(w)
                       if short_name(k).startswith(LIB_KERNEL_PREFIXES))
        rd = sum(_median(f[k]) * fs * 1024.0 for k in names if k in f)
        wr = sum(_median(w[k]) * wsc * 1024.0 for k in names if k in w)
        short = ", ".join(sorted({short_name(k) for k in names}))
        alg = rec["algorithmic_bytes"]
        lines.append(f"| {label} | {short} | {rd / 1e6:.1f} | {wr / 1e6:.1f} | "
                     f"{rd + wr:.4g} | {alg:.4g} | {(rd + wr) / alg:.3f} |")
    with open(out_md, "w") as fh:
        fh.write("\n".join(lines) + "\n")


def _counter_by_launch(run_dir, counter, name_part):
    """{grid size: [per-dispatch values]} of one counter for the kernels whose
    name contains name_part (the c5 products share one kernel name and differ
    in their grids)."""
    vals = defaultdict(list)
    for r in _rows(os.path.join(run_dir, "run_counter_collection.csv")):
        if r["Counter_Name"] == counter and name_part in r["Kernel_Name"]:
            vals[int(r["Grid_Size"])].append(float(r["Counter_Value"]))
    return vals


# The c5 products by grid size (256 lanes per 256 x 256 tile, or per half tile
# in the last round; on 256 CUs y's 1376 tiles run as 1280 whole tiles and
# 2 x 96 halves): their algorithmic bytes, A + B read once and C written once.
C5_PRODUCTS = {
    32 * 43 * 256: ("y = h W", 8192 * 4096 * 2 + 4096 * 11008 * 2, 8192 * 11008 * 2),
    (1280 + 2 * 96) * 256: ("y = h W", 8192 * 4096 * 2 + 4096 * 11008 * 2, 8192 * 11008 * 2),
    32 * 16 * 256: ("dh = dy W^T", 8192 * 11008 * 2 + 4096 * 11008 * 2, 8192 * 4096 * 2),
    16 * 43 * 256: ("dW = h^T dy", 8192 * 4096 * 2 + 8192 * 11008 * 2, 4096 * 11008 * 4),
}


def write_gemm_traffic_summary(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir, copy_mib,
                               out_md, command, name_part="gemm_nt_direct"):
    """HBM bytes per launch of each c5 product (median over its dispatches),
    against the bytes of its operands and result."""
    _, fs, ws = traffic(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir, copy_mib)
    f = _counter_by_launch(fetch_dir, "FETCH_SIZE", name_part)
    w = _counter_by_launch(write_dir, "WRITE_SIZE", name_part)
    lines = ["# HBM traffic per launch of the c5 products (bf16 GEMM)", "",
             "Commands (each counter in its own run):", "", "```", command, "```", "",
             f"Counter scale from a {copy_mib} MiB device copy (`bench.py --copy-probe "
             f"{copy_mib}`): FETCH_SIZE x {fs:.4f}, WRITE_SIZE x {ws:.4f}. Algorithmic bytes: "
             "A and B read once, C written once.", "",
             "| product | grid | launches | read MB | write MB | algorithmic read MB | "
             "algorithmic write MB | read ratio | write ratio |",
             "|---|---|---|---|---|---|---|---|---|"]
    for grid in sorted(set(f) | set(w)):
        name, ar, aw = C5_PRODUCTS.get(grid, (f"grid {grid}", 0, 0))
        rd = _median(f[grid]) * fs * 1024.0 if grid in f else 0.0
        wr = _median(w[grid]) * ws * 1024.0 if grid in w else 0.0
        n = max(len(f.get(grid, [])), len(w.get(grid, [])))
        lines.append(f"| {name} | {grid} | {n} | {rd / 1e6:.1f} | {wr / 1e6:.1f} | "
                     f"{ar / 1e6:.1f} | {aw / 1e6:.1f} | {rd / ar if ar else 0:.3f} | "
                     f"{wr / aw if aw else 0:.3f} |")
    with open(out_md, "w") as fh:
        fh.write("\n".join(lines) + "\n")


def write_mfma_summary(counter_csv, out_md, command, simds=1024, clock_ghz=2.4):
    per = defaultdict(lambda: defaultdict(float))
    disp = defaultdict(dict)
    for r in _rows(counter_csv):
        d = disp[r["Dispatch_Id"]]
        d["key"] = (short_name(r["Kernel_Name"]), r["Grid_Size"], r["Workgroup_Size"])
        d[r["Counter_Name"]] = float(r["Counter_Value"])
        d["ns"] = float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
    for d in disp.values():
        if d.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0) <= 0:
            continue
        acc = per[d["key"]]
        acc["n"] += 1
        for c in ("SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_LDS_BANK_CONFLICT",
                  "SQ_LDS_IDX_ACTIVE", "ns"):
            acc[c] += d.get(c, 0.0)
    lines = ["# MFMA use of the bf16 GEMM launches (rocprofv3 counters)", "", "Command:", "",
             "```", command, "```", "",
             f"flops = 512 x SQ_INSTS_VALU_MFMA_MOPS_BF16; MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / "
             f"({simds} SIMDs x {clock_ghz} GHz) as a share of the kernel's duration in the "
             "counter run; LDS conflict = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE.", "",
             "| kernel | grid | workgroup | launches | avg us | GFLOP | TFLOP/s | MFMA busy | "
             "LDS conflict |", "|---|---|---|---|---|---|---|---|---|"]
    for (name, grid, wg), a in sorted(per.items(), key=lambda kv: (kv[0][0], kv[0][1])):
        n = a["n"]
        us = a["ns"] / n / 1e3
        flops = 512.0 * a["SQ_INSTS_VALU_MFMA_MOPS_BF16"] / n
        busy_us = a["SQ_VALU_MFMA_BUSY_CYCLES"] / n / simds / (clock_ghz * 1e3)
        lds = a["SQ_LDS_BANK_CONFLICT"] / a["SQ_LDS_IDX_ACTIVE"] if a["SQ_LDS_IDX_ACTIVE"] else 0.0
        lines.append(f"| {name} | {grid} | {wg} | {int(n)} | {us:.1f} | {flops / 1e9:.1f} | "
                     f"{flops / (us * 1e-6) / 1e12:.0f} | {100 * busy_us / us:.1f} % | "
                     f"{100 * lds:.2f} % |")
    with open(out_md, "w") as fh:
        fh.write("\n".join(lines) + "\n")


def _cfg_label(r):
    return (f"{r['config']['workload'].split(':')[0]} {r['config']['rows']}x"
            f"{r['config']['cols']} {r['dtype']}")


def _gpu_state_line(gs):
    """The shader clock and board power bench.py read from sysfs around a timed
    region, as one sentence (None when the record has none)."""
    if not gs or not gs.get("after_timed"):
        return None
    b, a = gs.get("before_timed") or {}, gs["after_timed"]
    return (f"GPU state (sysfs): shader clock {b.get('sclk_mhz', '-')} -> {a.get('sclk_mhz', '-')}"
            f" MHz, board power {b.get('power_w', '-')} -> {a.get('power_w', '-')} W (during the "
            "last warm-up steps -> right after the timed steps).")


def write_bench_summary(jsonl, out_md, command):
    """Tables of bench.py's JSON lines (RMSNorm configurations, c5, row ops)."""
    recs = [json.loads(ln) for ln in open(jsonl) if ln.strip().startswith("{")]
    lines = ["# bench.py results (MI355X, one GPU)", "", "Command:", "", "```", command, "```", "",
             "Kernel times are HIP events on the launch stream, averaged over the timed steps; "
             "GB/s are algorithmic bytes over those times; % is of the 8 TB/s HBM peak.", ""]
    norm = [r for r in recs if r.get("unit") == "GB/s" and "fwd" in r.get("kernels", {})
            and r["metric"].startswith("RMSNorm")]
    if norm:
        lines += ["## RMSNorm layer fwd + VJP", "",
                  "| config | fwd+bwd GB/s | % of peak | step us | fwd us | fwd % | bwd us | bwd % "
                  "| CPU GB/s (threads) | CPU 1-thread GB/s |",
                  "|---|---|---|---|---|---|---|---|---|---|"]
        for r in norm:
            k = r["kernels"]
            cpu = r.get("cpu_baseline") or {}
            one = (cpu.get("modes") or {}).get("single_thread") or {}
            lines.append(f"| {_cfg_label(r)} | {r['value']:.0f} | "
                         f"{100 * r['value'] / 8000:.1f} | {1e3 * r['ms_per_step']:.1f} | "
                         f"{1e3 * k['fwd']['avg_ms']:.1f} | "
                         f"{100 * k['fwd']['frac']:.1f} | {1e3 * k['bwd']['avg_ms']:.1f} | "
                         f"{100 * k['bwd']['frac']:.1f} | "
                         f"{cpu.get('value', '-')} ({cpu.get('cores', '-')}) | "
                         f"{one.get('gbs', '-')} |")
        lines.append("")
        graphed = [r for r in norm if r.get("graph")]
        if graphed:
            lines += ["The same calls captured once into a HIP graph and replayed (best of 5 "
                      "replays of the timed number of steps): the GPU's own time, without the "
                      "host's cost of launching each call from Python. Where the two tables "
                      "differ, the eager step above is bound by the host's launch rate.", "",
                      "| config | step us | GB/s | % of peak | fwd us | bwd us | fwd+bwd us "
                      "(separate graphs) | step us, one set |", "|---|---|---|---|---|---|---|---|"]
            for r in graphed:
                gr = r["graph"]
                one = gr.get("ms_per_step_one_set")
                lines.append(f"| {_cfg_label(r)} | {1e3 * gr['ms_per_step']:.1f} | "
                             f"{gr['gbs']:.0f} | {gr['pct_of_hbm_peak']:.1f} | "
                             f"{1e3 * gr['fwd_ms']:.1f} | {1e3 * gr['bwd_ms']:.1f} | "
                             f"{1e3 * (gr['fwd_ms'] + gr['bwd_ms']):.1f} | "
                             f"{'-' if one is None else f'{1e3 * one:.1f}'} |")
            lines += ["", "The steps rotate over min(8, ceil(2 GiB / one set's bytes)) sets of "
                      "tensors, so a small configuration's call does not find its inputs in L2 "
                      "(4 MB per XCD). \"One set\" replays the same steps on a single set, "
                      "whose tensors then stay in L2 and the Infinity Cache, as a layer's input "
                      "does when the previous op has just written it.", ""]
        hosts = {json.dumps(r["cpu_baseline"]["host"], sort_keys=True) for r in norm
                 if r.get("cpu_baseline") and r["cpu_baseline"].get("host")}
        for h in hosts:
            h = json.loads(h)
            lines += [f"CPU baseline host: {h.get('cpu_model')}, hardware_concurrency "
                      f"{h.get('hardware_concurrency')}, {h.get('usable_cpus')} usable CPUs, "
                      f"last-level cache {h.get('llc_bytes')} bytes. The CPU figure times the "
                      "oracle's op-by-op restatement of the reference path (a restatement, not "
                      "OwnTensor) on a row sample of at least the last-level cache per tensor, "
                      "median of 5 runs.", ""]
    rows = [r for r in recs if r.get("unit") == "GB/s" and not r["metric"].startswith("RMSNorm")]
    if rows:
        lines += ["## Row ops on the same skeleton", "",
                  "| workload | kernel | us | GB/s | % of peak | CPU oracle GB/s |",
                  "|---|---|---|---|---|---|"]
        for r in rows:
            cpu = r.get("cpu_baseline")
            for name, k in r["kernels"].items():
                lines.append(f"| {r['config']['workload']} | {name} | {1e3 * k['avg_ms']:.1f} | "
                             f"{k['gbs']:.0f} | {100 * k['frac']:.1f} | "
                             f"{cpu['value'] if cpu else '-'} |")
        lines.append("")
    for r in recs:
        if r.get("unit") != "TFLOP/s":
            continue
        st, tb = r["stages_ms"], r["torch_hipblaslt_ms"]
        fl = r["config"]["gemm_flops_per_step"] / 3
        cpu = r.get("cpu_baseline") or {}
        lines += ["## RMSNorm + linear layer (c5)", "",
                  f"M, K, N = {r['config']['M']}, {r['config']['K']}, {r['config']['N']}; "
                  f"{r['value']} TFLOP/s over the three products "
                  f"({100 * r['roofline']['frac']:.1f} % of 2.5 PFLOP/s dense bf16); "
                  f"hipBLASLt on the same operands {r['torch_hipblaslt_tflops']} TFLOP/s; "
                  f"CPU oracle {cpu.get('value', '-')} TFLOP/s on {cpu.get('cores', '-')} "
                  f"threads.", "",
                  "In the layer step: each stage as the timed step runs it (products between "
                  "the RMSNorm kernels). Alone: the product repeated back to back, the way "
                  "hipBLASLt is timed.", "",
                  "| stage | in the layer step us | TFLOP/s | alone us | TFLOP/s | "
                  "hipBLASLt us | TFLOP/s |", "|---|---|---|---|---|---|---|"]
        alone = r.get("alone_ms", {})
        for name, ms in st.items():
            if name in tb:
                al = alone.get(name)
                al_cols = (f"{1e3 * al:.1f} | {fl / (al * 1e-3) / 1e12:.0f}" if al else "- | -")
                lines.append(f"| {name} | {1e3 * ms:.1f} | {fl / (ms * 1e-3) / 1e12:.0f} | "
                             f"{al_cols} | "
                             f"{1e3 * tb[name]:.1f} | {fl / (tb[name] * 1e-3) / 1e12:.0f} |")
            else:
                lines.append(f"| {name} | {1e3 * ms:.1f} | - | - | - | - | - |")
        lines.append("")
        state = _gpu_state_line(r.get("gpu_state"))
        if state:
            lines += [state + " The products run into the board's power limit, so their "
                      "speed follows the power this box allows.", ""]
    gstates = [(_cfg_label(r), _gpu_state_line((r.get("kernels") or {}).get("gpu_state")))
               for r in norm]
    gstates = [(c, g) for c, g in gstates if g]
    if gstates:
        lines += ["GPU state per RMSNorm configuration:", ""]
        lines += [f"- {c}: {g}" for c, g in gstates]
        lines.append("")
    with open(out_md, "w") as fh:
        fh.write("\n".join(lines) + "\n")


def write_probe_summary(jsonl, out_md, command):
    """Table of bench.py --stream-probe lines: GB/s per traffic mix, cache policy
    and grid (0 = one workgroup per 16 KiB chunk)."""
    recs = [json.loads(ln) for ln in open(jsonl) if ln.strip().startswith("{")]
    recs = [r for r in recs if "stream_probe" in r]
    grids = sorted({g for r in recs for g in r["gbs_by_grid"]}, key=int)
    lines = ["# HBM streaming probe (bench.py --stream-probe)", "", "Command:", "", "```",
             command, "```", "",
             f"{recs[0]['mib_per_buffer'] if recs else '?'} MiB per buffer, 16-byte slots; GB/s "
             "counts every byte read and written; HIP events on the launch stream. Grid 0 is "
             "one 256-lane workgroup per contiguous 16 KiB chunk (how the row kernels touch "
             "memory); the others are grid-stride loops of that many workgroups.", "",
             "| mix | non-temporal | " + " | ".join(f"grid {g}" for g in grids) +
             " | best % of 8 TB/s |", "|---|---|" + "---|" * len(grids) + "---|"]
    for r in recs:
        lines.append(f"| {r['stream_probe']} | {'yes' if r['nontemporal'] else 'no'} | " +
                     " | ".join(f"{r['gbs_by_grid'].get(g, '-')}" for g in grids) +
                     f" | {r['pct_of_hbm_peak']} |")
    with open(out_md, "w") as fh:
        fh.write("\n".join(lines) + "\n")


def write_mfma_probe_summary(jsonl, out_md, command):
    """Table of bench.py --mfma-probe lines: what the matrix cores sustain with
    the bf16 GEMM's inner loop (no global loads, no barriers), by operand
    content, with the shader clock the loop ran at."""
    recs = [json.loads(ln) for ln in open(jsonl) if ln.strip().startswith('{"mfma_probe"')]
    lines = ["# MFMA probe: the bf16 GEMM's inner loop without loads (bench.py --mfma-probe)", "",
             "Command:", "", "```", command, "```", "",
             "256 workgroups of 4 waves (one wave per SIMD, as `gemm_nt_direct_kernel`), each "
             "wave 16 `v_mfma_f32_32x32x16_bf16` accumulators (a 128 x 128 block), "
             f"{recs[0]['k_steps_per_wave'] if recs else '?'} 64-deep k-steps per wave. "
             "'lds': every substep's 8 fragments read from a 64 KiB LDS tile one substep "
             "ahead (the GEMM's LDS traffic and schedule); 'registers': MFMAs only; the "
             "'16x16x32' modes: the same block as 8 x 8 `v_mfma_f32_16x16x32_bf16` "
             "accumulators, 128 MFMAs per k-step, the same fragment bytes per k. "
             "TFLOP/s from HIP events; the shader clock and cycles per k-step from "
             "s_memtime / s_memrealtime (100 MHz) read by wave 0 of each workgroup around "
             "its loop (medians over workgroups). A k-step is 2048 cycles at the full issue "
             "rate of either instruction. Dense bf16 peak: 2500 TFLOP/s at 2.4 GHz.", "",
             "| mode | operand data | TFLOP/s | % of dense peak | shader GHz | cycles per k-step |",
             "|---|---|---|---|---|---|"]
    for r in recs:
        lines.append(f"| {r['mfma_probe']} | {r['data']} | {r['tflops']} | "
                     f"{r['pct_of_dense_peak']} | {r['shader_ghz']} | {r['cycles_per_k_step']} |")
    with open(out_md, "w") as fh:
        fh.write("\n".join(lines) + "\n")


def write_gemm_f32_summary(jsonl, out_md, command):
    """Table of bench.py --gemm-f32 lines: agk_gemm_f32 against torch's fp32
    matmul in the four operand layouts."""
    recs = [json.loads(ln) for ln in open(jsonl) if ln.strip().startswith('{"gemm_f32"')]
    lays = ("AB", "ABt", "AtB", "AtBt")
    lines = ["# fp32 GEMM (agk_gemm_f32, bench.py --gemm-f32)", "", "Command:", "", "```",
             command, "```", "",
             "TFLOP/s from HIP events on the launch stream (warm-up calls first), "
             "agk_gemm_f32 / torch.matmul in fp32 on the same operands. Layouts: A [M, K] or "
             "At = A given as [K, M]; B [K, N] or Bt = B given as [N, K]. fp32 matrix peak "
             "157.3 TFLOP/s.", "",
             "| M x N x K | " + " | ".join(lays) + " |", "|---|" + "---|" * len(lays)]
    for r in recs:
        lines.append(f"| {r['gemm_f32']} | " + " | ".join(
            f"{r['tflops'][k]} / {r['torch_tflops'][k]}" for k in lays) + " |")
    with open(out_md, "w") as fh:
        fh.write("\n".join(lines) + "\n")


def _wide_bwd_path(plan):
    """The backward path a launch plan names (agk_rmsnorm_launch_plan)."""
    if plan["tpr"] > 0 and plan["g"] == 0:
        return f"team of {plan['tpr'] // 256}"
    if plan["tpr"] == 1024 and plan["nblk"] == 256:
        return "one pass"
    if plan["tpr"] == 0 and plan["nv"] > 0:
        return "split"
    return "resident" if plan["tpr"] > 0 else "looped"


def write_wide_summary(jsonl, out_md, command):
    """Table of bench.py --wide lines: the wide paths against the
    one-workgroup-per-row kernels per shape (graph-replayed us and GB/s)."""
    recs = [json.loads(ln) for ln in open(jsonl) if ln.strip().startswith('{"wide_rows"')]
    lines = ["# Rows wider than the register-resident kernels (MI355X, one GPU)", "",
             "Command:", "", "```", command, "```", "",
             "Each call captured into a HIP graph and replayed (GPU time per call, best of 5 "
             "replays). Forward: out of place (the split path for rows too wide for "
             "registers: x read twice), the same with a workspace (agk_rmsnorm_fwd_ws, "
             "'fwd ws': the team kernel where 'fwd ws path' names it -- a row over that many "
             "workgroups exchanging partial sums, x read once -- else the same kernels), "
             "and in place (y = x keeps one workgroup per row). Backward "
             "(dx and dgamma) and dx alone: as the library takes them with a workspace "
             "('path': the one-pass kernel for rows of up to 32768 columns from 256 rows, "
             "the team kernel -- a row over that many workgroups exchanging partial sums -- "
             "for other aligned rows of up to 1M columns), then the same calls with the team "
             "kernel switched off (the split path: x and dy read twice), and dx alone "
             "without a workspace (looped). GB/s: algorithmic bytes (forward 2 tensors, "
             "backward 3) over the time; % of 8 TB/s in brackets.",
             "",
             "| shape | fwd ws path | bwd path | fwd split us | fwd ws us | fwd in place us | "
             "bwd us | bwd split us | bwd dx us | bwd dx split us | bwd dx looped us | "
             "fwd split GB/s | fwd ws GB/s | bwd GB/s | bwd split GB/s |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for r in recs:
        u, g = r["us"], r["gbs"]
        fwp = r.get("fwd_ws_plan", {})
        fpath = (f"team of {fwp['tpr'] // 256}" if fwp.get("g") == 0 and fwp.get("tpr")
                 else ("split" if r["fwd_plan"]["tpr"] == 0 else "resident"))
        lines.append(f"| {r['wide_rows']} | {fpath} | {_wide_bwd_path(r['bwd_plan'])} | "
                     f"{u['fwd_split']} | {u['fwd_ws']} | {u['fwd_in_place']} | {u['bwd']} | "
                     f"{u['bwd_split']} | {u['bwd_dx']} | {u['bwd_dx_split']} | "
                     f"{u['bwd_dx_looped']} | "
                     f"{g['fwd_split']:.0f} ({g['fwd_split'] / 80:.1f} %) | "
                     f"{g['fwd_ws']:.0f} ({g['fwd_ws'] / 80:.1f} %) | "
                     f"{g['bwd']:.0f} ({g['bwd'] / 80:.1f} %) | "
                     f"{g['bwd_split']:.0f} ({g['bwd_split'] / 80:.1f} %) |")
    ro = [json.loads(ln) for ln in open(jsonl) if ln.strip().startswith('{"wide_rowops"')]
    if ro:
        lines += ["", "## Softmax and log-sum-exp at vocabulary widths", "",
                  "Graph-replayed µs per call on the same values in three layouts: 16-byte "
                  "aligned tensors / every tensor one element off a 16-byte boundary (the "
                  "16-byte looped kernel's head/body/tail form; at 50257 columns every row "
                  "is off a boundary, so both take it) / inputs off and outputs aligned (the "
                  "element-wise looped kernel; log-sum-exp forward has no row output, so "
                  "'-'). % of 8 TB/s for the first layout (algorithmic bytes: softmax forward "
                  "2 tensors, backward 3, log-sum-exp forward 1, backward 2). The 16-byte "
                  "kernel computes the row maximum and the sum of exponentials in one online "
                  "pass. 'log-sum-exp bwd from value' is agk_logsumexp_bwd_from_value: "
                  "dz = dy * exp(z - lse) with the forward's fp32 lse (one read of z, one "
                  "write of dz; what the graph layer's vjp_LogSumExpRow runs); 'log-sum-exp "
                  "bwd' recomputes the row maximum and sum as the reference's rule does.", "",
                  "Softmax forward and backward and the log-sum-exp backward are called "
                  "with a workspace (agk_*_ws): rows of more than 8192 16-byte slots, and for "
                  "the softmax backward rows off a 16-byte boundary of more than 2048, take "
                  "the team kernel "
                  "('team': workgroups per row for softmax fwd / softmax bwd / log-sum-exp bwd "
                  "in the aligned and offset layouts, 0 for none; a row over that many "
                  "workgroups that exchange partial sums, so each input row is read once). "
                  "The 'no workspace' columns time the same calls without one (the "
                  "one-workgroup-per-row kernels) in the first two layouts.", "",
                  "| shape | team | softmax fwd | softmax bwd | log-sum-exp fwd | "
                  "log-sum-exp bwd | log-sum-exp bwd from value | softmax fwd, no workspace | "
                  "softmax bwd, no workspace | log-sum-exp bwd, no workspace |",
                  "|---|---|---|---|---|---|---|---|---|---|"]
        for r in ro:
            u, g = r["us"], r["gbs"]
            cells = []
            for k in ("softmax_fwd", "softmax_bwd", "logsumexp_fwd", "logsumexp_bwd",
                      "logsumexp_bwd_from_value"):
                if k + "_vec" not in u:
                    cells.append("-")
                    continue
                sc = u.get(k + "_scalar", "-")
                cells.append(f"{u[k + '_vec']} / {u[k + '_offset']} / {sc} "
                             f"({g[k + '_vec'] / 80:.1f} %)")
            for k in ("softmax_fwd_nows", "softmax_bwd_nows", "logsumexp_bwd_nows"):
                if k + "_vec" not in u:
                    cells.append("-")
                    continue
                cells.append(f"{u[k + '_vec']} / {u[k + '_offset']} "
                             f"({g[k + '_vec'] / 80:.1f} %)")
            team = r.get("team")
            tcell = ("; ".join(f"{lay}: " + "/".join(str(team[lay][op]["parts"]) for op in
                                                    ("softmax_fwd", "softmax_bwd",
                                                     "logsumexp_bwd")) for lay in
                               ("aligned", "offset")) if team else "-")
            lines.append(f"| {r['wide_rowops']} | {tcell} | " + " | ".join(cells) + " |")
    with open(out_md, "w") as fh:
        fh.write("\n".join(lines) + "\n")


def main(argv):
    if len(argv) >= 4 and argv[0] == "wide":
        write_wide_summary(argv[1], argv[2], argv[3])
    elif len(argv) >= 4 and argv[0] == "trace":
        write_trace_summary(argv[1], argv[2], argv[3])
    elif len(argv) >= 4 and argv[0] == "probe":
        write_probe_summary(argv[1], argv[2], argv[3])
    elif len(argv) >= 4 and argv[0] == "mfma-probe":
        write_mfma_probe_summary(argv[1], argv[2], argv[3])
    elif len(argv) >= 4 and argv[0] == "gemm-f32":
        write_gemm_f32_summary(argv[1], argv[2], argv[3])
    elif len(argv) >= 4 and argv[0] == "bench":
        write_bench_summary(argv[1], argv[2], argv[3])
    elif len(argv) >= 4 and argv[0] == "mfma":
        write_mfma_summary(argv[1], argv[2], argv[3])
    elif len(argv) >= 8 and argv[0] == "gemm-traffic":
        write_gemm_traffic_summary(argv[1], argv[2], argv[3], argv[4], int(argv[5]), argv[6],
                                   argv[7])
    elif len(argv) >= 7 and argv[0] == "wide-traffic":
        runs = [tuple(a.split(",")) for a in argv[6:]]
        write_wide_traffic_summary(argv[1], argv[2], int(argv[3]), argv[4], argv[5], runs)
    elif len(argv) >= 9 and argv[0] == "traffic":
        write_traffic_summary(argv[1], argv[2], argv[3], argv[4], int(argv[5]), argv[6],
                              argv[7], argv[8])
    else:
        sys.stderr.write(__doc__)
        return 2
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))

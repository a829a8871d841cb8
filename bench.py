#!/usr/bin/env python3
"""RMSNorm layer forward + VJP on one MI355X, through the C ABI.

One step = agk_rmsnorm_fwd (y, inv_rms) + agk_rmsnorm_bwd (dx, dgamma: the
backward kernel and the dgamma column reduction) over one batch of the
configuration, inputs resident in HBM before the timed region starts.

  value        algorithmic bytes per step / wall time per step (GB/s), with
               bytes = 5*R*D*s + 2*D*s_gamma + 2*R*4 + D*4
  roofline     the backward launch (dominant: 3 of the 5 passes), its
               algorithmic bytes / its average duration from HIP events on
               the stream it runs on, against MI355X's 8 TB/s HBM peak
  cpu_baseline the CPU oracle (op-by-op restatement of the reference path,
               OpenMP over the host cores) on a bounded row sample

Default workload: configuration c2, x [32,2048,4096] fp32 (65,536 rows of
4096).  --config selects another configuration (c1..c4c) for exploration;
--gpus above 1 is refused (this build runs on one GPU).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = ("RMSNorm fwd+bwd achieved HBM GB/s (% of peak) at [32,2048,4096]; vs host CPU")
HBM_PEAK_GBS = 8000.0
DEFAULT_CONFIG = "c2"


class TimingEvent:
    """A HIP event for timing only, recorded on the stream the kernels run on.

    Created with hipEventDisableSystemFence: recording it adds no system-scope
    fence (cache writeback and invalidate), which with torch.cuda.Event leaves
    the GPU idle for ~5 us around every record and would count against the
    step.  It comes from the HIP runtime torch itself loaded (opening the same
    file returns the loaded object), so torch's stream handles are valid for
    it.  Same interface as torch.cuda.Event: record(stream), elapsed_time(end).
    """

    _hip = None
    _DISABLE_SYSTEM_FENCE = 0x20000000

    @classmethod
    def _runtime(cls):
        if cls._hip is None:
            import ctypes

            import torch
            hip = ctypes.CDLL(os.path.join(os.path.dirname(torch.__file__), "lib",
                                           "libamdhip64.so"))
            hip.hipEventCreateWithFlags.argtypes = [ctypes.c_void_p, ctypes.c_uint]
            hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            hip.hipEventElapsedTime.argtypes = [ctypes.c_void_p, ctypes.c_void_p,
                                                ctypes.c_void_p]
            hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
            cls._hip = hip
        return cls._hip

    def __init__(self):
        import ctypes
        self._ctypes = ctypes
        self._ev = ctypes.c_void_p()
        rc = self._runtime().hipEventCreateWithFlags(ctypes.byref(self._ev),
                                                     self._DISABLE_SYSTEM_FENCE)
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")

    def record(self, stream):
        rc = self._runtime().hipEventRecord(self._ev, self._ctypes.c_void_p(stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_time(self, end):
        ms = self._ctypes.c_float()
        rc = self._runtime().hipEventElapsedTime(self._ctypes.byref(ms), self._ev, end._ev)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def __del__(self):
        if self._hip is not None and self._ev:
            self._hip.hipEventDestroy(self._ev)


def _bench_lib():
    """libagk_bench.so: the benchmark's measurement probes (agk_probe_stream,
    agk_probe_mfma; cgadimpl_amd/csrc/agk_bench.h), built beside the kernel
    library but not part of it."""
    import ctypes

    import cgadimpl_amd as agk
    global _BENCH_LIB
    if _BENCH_LIB is None:
        path = os.path.join(agk.LIB_DIR, "libagk_bench.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run __graft_entry__.build() first")
        agk.lib()  # loads torch's HIP runtime first (see cgadimpl_amd.lib)
        h = ctypes.CDLL(path)
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        h.agk_probe_stream.restype = I
        h.agk_probe_stream.argtypes = [P, P, P, P, I64, I, I, I, I, P]
        h.agk_probe_mfma.restype = I
        h.agk_probe_mfma.argtypes = [P, P, P, I, I, I, P]
        _BENCH_LIB = h
    return _BENCH_LIB


_BENCH_LIB = None


def probe_stream(a, b, c, d, nbytes, reads, writes, nontemporal, grid, stream):
    """agk_probe_stream: reads `reads` buffers, writes `writes` (a diagnostic)."""
    rc = _bench_lib().agk_probe_stream(
        a.data_ptr(), b.data_ptr() if b is not None else None, c.data_ptr(),
        d.data_ptr() if d is not None else None, int(nbytes), int(reads), int(writes),
        int(bool(nontemporal)), int(grid), stream.cuda_stream)
    if rc != 0:
        raise RuntimeError(f"agk_probe_stream failed ({rc})")


def gpu_state():
    """The GPU's shader and memory clocks, board power and temperatures from
    sysfs (amdgpu's hwmon and pp_dpm files) at the moment of the call, for the
    device torch runs on; None for what this host does not expose.  Read before
    and after a timed region, so a slow box shows up as a slow box."""
    import glob
    import torch
    out = {"sclk_mhz": None, "mclk_mhz": None, "power_w": None, "temp_edge_c": None,
           "temp_junction_c": None, "temp_mem_c": None, "source": None}
    dev_dir = None
    try:
        p = torch.cuda.get_device_properties(torch.cuda.current_device())
        dom = getattr(p, "pci_domain_id", None)
        bus = getattr(p, "pci_bus_id", None)
        slot = getattr(p, "pci_device_id", None)
        if bus is not None and slot is not None:
            cand = "/sys/bus/pci/devices/%04x:%02x:%02x.0" % (dom or 0, bus, slot)
            if os.path.isdir(cand):
                dev_dir = cand
    except Exception:  # noqa: BLE001 - diagnostic only
        pass
    if dev_dir is None:  # one AMD GPU visible in sysfs: take it
        cards = [d for d in glob.glob("/sys/class/drm/card*/device")
                 if os.path.exists(os.path.join(d, "pp_dpm_sclk"))]
        if len(set(os.path.realpath(c) for c in cards)) == 1:
            dev_dir = cards[0]
    if dev_dir is None:
        out["source"] = "no sysfs device matched"
        return out
    out["source"] = os.path.realpath(dev_dir)

    def read(path):
        try:
            with open(path) as f:
                return f.read().strip()
        except OSError:
            return None

    def dpm_current(name):
        txt = read(os.path.join(dev_dir, name))
        if not txt:
            return None
        for ln in txt.splitlines():
            if ln.rstrip().endswith("*"):
                num = "".join(ch for ch in ln.split(":", 1)[-1] if ch.isdigit())
                return int(num) if num else None
        return None

    hw = sorted(glob.glob(os.path.join(dev_dir, "hwmon", "hwmon*")))
    h = hw[0] if hw else None
    if h:
        f1 = read(os.path.join(h, "freq1_input"))
        f2 = read(os.path.join(h, "freq2_input"))
        out["sclk_mhz"] = round(int(f1) / 1e6) if f1 and f1.isdigit() else None
        out["mclk_mhz"] = round(int(f2) / 1e6) if f2 and f2.isdigit() else None
        for name in ("power1_average", "power1_input"):
            v = read(os.path.join(h, name))
            if v and v.isdigit():
                out["power_w"] = round(int(v) / 1e6, 1)
                break
        for key, name in (("temp_edge_c", "temp1_input"), ("temp_junction_c", "temp2_input"),
                          ("temp_mem_c", "temp3_input")):
            v = read(os.path.join(h, name))
            out[key] = round(int(v) / 1e3, 1) if v and v.lstrip("-").isdigit() else None
    if out["sclk_mhz"] is None:
        out["sclk_mhz"] = dpm_current("pp_dpm_sclk")
    if out["mclk_mhz"] is None:
        out["mclk_mhz"] = dpm_current("pp_dpm_mclk")
    return out


def graph_replay_ms(body, n, reps=5):
    """Milliseconds per body() when n calls of it are captured once into a HIP
    graph (torch.cuda.CUDAGraph) and the graph is replayed: the GPU's time for
    the calls without the host's per-call launch cost.  body(i, stream) issues
    call i on `stream`.  Best of `reps` replays, timed with HIP events on the
    replay stream after one untimed replay."""
    import torch
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        cs = torch.cuda.current_stream()
        for i in range(n):
            body(i, cs)
    stream = torch.cuda.current_stream()
    graph.replay()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        e0, e1 = TimingEvent(), TimingEvent()
        e0.record(stream)
        graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1))
    del graph
    return best / n


def _device_inputs(cfg, dev, seed):
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    R, D = cfg.rows, cfg.cols
    x = torch.randn((R, D), generator=gen, device=dev) * cfg.x_std
    g = torch.rand(D, generator=gen, device=dev) + 0.5
    dy = torch.randn((R, D), generator=gen, device=dev)
    if cfg.outlier_p > 0:
        mask = torch.rand((R, D), generator=gen, device=dev) < cfg.outlier_p
        x = torch.where(mask, x * cfg.outlier_scale, x)
        del mask
    if cfg.dtype == "bf16":
        x, g, dy = x.bfloat16(), g.bfloat16(), dy.bfloat16()
    return x.contiguous(), g.contiguous(), dy.contiguous()


def _traffic(config_name):
    """HBM bytes per backward call (FETCH_SIZE + WRITE_SIZE, scaled by a copy of
    known size) from the committed rocprofv3 summary of this configuration, and
    where it came from.  A summary whose kernel-source hash differs from the
    current sources describes other kernels: its figure is not used (None)."""
    from cgadimpl_amd import profiling
    path = os.path.join(ROOT, "profiles", f"rmsnorm_{config_name}_hbm_traffic.json")
    if not os.path.exists(path):
        return None, "no rocprofv3 traffic summary for this configuration"
    with open(path) as fh:
        rec = json.load(fh)
    rel = os.path.relpath(path, ROOT)
    if rec.get("kernel_source_sha256") != profiling.kernel_source_hash(ROOT):
        return None, f"{rel} was measured on other kernel sources (stale, not used)"
    return rec.get("bwd_hbm_bytes_per_launch"), f"{rel} (kernel sources match)"


def _bwd_kernels(agk, rows, cols, dtype):
    """The kernels one agk_rmsnorm_bwd call of these sizes launches."""
    p = agk.launch_plan(rows, cols, agk.AGK_F32 if dtype == "f32" else agk.AGK_BF16, True)
    if p["tpr"] == 0 and p["nv"] > 0:
        return ("wide_row_stats + wide_row_finish + wide_bwd_tiles"
                + (" + dgamma_finalize" if p["nblk"] else ""))
    if p["tpr"] == 0:
        return "rms_bwd_looped + dgamma_finalize"
    if cols > 16384 and p["tpr"] == 1024 and p["nv"] * (4 if dtype == "f32" else 8) * 1024 > 16384:
        return "wide_bwd_resident + dgamma_finalize"
    if p["nblk"] == 0:
        return "bwd_fewrows: row and column workgroups, one launch"
    return "rms_bwd_resident + dgamma_finalize"


def host_info():
    """The host's CPU: model string, logical CPU count (what C++'s
    std::thread::hardware_concurrency() reports), the CPUs this process may run
    on, and the last-level cache size, read from /proc and /sys."""
    model = None
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    llc = None
    base = "/sys/devices/system/cpu/cpu0/cache"
    try:
        for idx in sorted(os.listdir(base)):
            try:
                with open(os.path.join(base, idx, "level")) as fh:
                    level = int(fh.read())
                with open(os.path.join(base, idx, "size")) as fh:
                    txt = fh.read().strip().upper()
                size = int(txt.rstrip("KMG")) * {"K": 1 << 10, "M": 1 << 20, "G": 1 << 30}.get(
                    txt[-1], 1)
                if llc is None or level >= llc[0]:
                    llc = (level, size)
            except (OSError, ValueError):
                continue
    except OSError:
        pass
    return {"cpu_model": model, "hardware_concurrency": os.cpu_count(),
            "usable_cpus": len(os.sched_getaffinity(0)),
            "llc_bytes": llc[1] if llc else None}


CPU_SAMPLE_MIN_BYTES = 64 << 20  # per tensor, and at least the last-level cache
CPU_RUNS = 5                     # timed runs per mode; the median is reported


def _keep_freed_memory():
    """Asks glibc malloc to serve large blocks from its heap and keep freed
    memory (mallopt M_MMAP_MAX = 0, M_TRIM_THRESHOLD = max), so the
    restatement's per-call intermediates are not re-faulted from the kernel on
    every run: that would time page faults (half the run time on the build
    host), not the CPU path."""
    import ctypes
    try:
        libc = ctypes.CDLL("libc.so.6")
        libc.mallopt(-4, 0)            # M_MMAP_MAX
        libc.mallopt(-1, 0x7fffffff)   # M_TRIM_THRESHOLD
    except OSError:
        pass


def cpu_baseline(cfg, seconds=None):
    """The CPU oracle on a bounded sample of the configuration, timed on this host.

    What is timed is the oracle's restatement of the reference's CPU op
    sequence (normalization.cpp:24-27, arithmetic.cpp:32, autodiff_vjp_ops.cpp:
    15-35,54-59,368-377, graph.cpp:46), every intermediate materialised as the
    reference graph does: the reference itself cannot be built here (its
    tensor library is an empty submodule), so this times a restatement, not
    OwnTensor.  The sample is whole rows of the configuration's inputs (same
    generator and distributions), at least the host's last-level cache and
    CPU_SAMPLE_MIN_BYTES per tensor, so the restatement's working set (about
    ten tensors) streams from DRAM.  Two modes: one thread, and every CPU this
    process may use (OpenMP); each reports the median of CPU_RUNS timed runs
    after one untimed run.  (`seconds` is unused: the sample, not a time
    budget, fixes the work.)
    """
    import oracle
    from cgadimpl_amd import configs
    info = host_info()
    R, D, s = cfg.rows, cfg.cols, cfg.storage_bytes
    per_tensor = max(CPU_SAMPLE_MIN_BYTES, info["llc_bytes"] or 0)
    rows = max(1, min(R, -(-per_tensor // (D * s))))
    x, g, dy = configs.config_inputs(cfg, (rows, D))
    _keep_freed_memory()
    sample_bytes = 5 * rows * D * s + 2 * D * s + 2 * rows * 4 + D * 4

    def one():
        _, inv = oracle.fwd(x, g, cfg.eps)
        oracle.bwd(x, g, inv, dy)

    modes = {}
    for mode, threads in (("single_thread", 1), ("all_cpus", info["usable_cpus"])):
        oracle.set_threads(threads)
        one()  # untimed: page-in, thread pool
        times = []
        for _ in range(CPU_RUNS):
            t0 = time.perf_counter()
            one()
            times.append(time.perf_counter() - t0)
        med = sorted(times)[len(times) // 2]
        modes[mode] = {"threads": threads, "median_s": round(med, 4),
                       "gbs": round(sample_bytes / med / 1e9, 3),
                       "rows_per_s": round(rows / med, 1)}
    best = modes["all_cpus"]
    return {
        "value": best["gbs"],
        "unit": "GB/s",
        "cores": best["threads"],
        "kind": "port",
        "sample": (f"{rows} of {R} rows x {D} {cfg.dtype} "
                   f"({rows * D * s / 2**20:.0f} MiB per tensor), fwd+VJP of the "
                   f"oracle's op-by-op restatement of the reference CPU path (every "
                   f"intermediate materialised; a restatement, not OwnTensor), median of "
                   f"{CPU_RUNS} runs on {best['threads']} OpenMP threads; rows/s "
                   f"{best['rows_per_s']:.4g}"),
        "modes": modes,
        "host": info,
    }


def run(cfg_name, steps, warmup, cpu_seconds):
    import torch

    import cgadimpl_amd as agk
    from cgadimpl_amd import configs

    cfg = configs.CONFIGS[cfg_name]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    R, D = cfg.rows, cfg.cols
    per_set = (4 if cfg.dtype == "f32" else 2) * R * D * 4  # x, dy, y, dx
    # rotate input/output sets so that small configurations are not served
    # from the 256 MB Infinity Cache between steps
    nsets = max(1, min(8, math.ceil((2 << 30) / per_set)))
    sets = []
    for i in range(nsets):
        x, g, dy = _device_inputs(cfg, dev, cfg.seed + i)
        y = torch.empty_like(x)
        inv = torch.empty(R, dtype=torch.float32, device=dev)
        dx = torch.empty_like(x)
        dg = torch.empty(D, dtype=torch.float32, device=dev)
        sets.append((x, g, dy, y, inv, dx, dg))
    ws = torch.empty(max(1, agk.rmsnorm_bwd_workspace_bytes(R, D)), dtype=torch.uint8,
                     device=dev)
    stream = torch.cuda.current_stream()

    def fwd(i, st):
        x, g, dy, y, inv, dx, dg = sets[i % nsets]
        agk.rmsnorm_fwd(x, g, cfg.eps, y=y, inv_rms=inv, stream=st)

    def bwd(i, st):
        x, g, dy, y, inv, dx, dg = sets[i % nsets]
        agk.rmsnorm_bwd(x, g, inv, dy, dx=dx, dgamma=dg, workspace=ws, stream=st)

    def step(i, ev_fwd=None, ev_bwd=None):
        if ev_fwd is not None:
            ev_fwd[0].record(stream)
        fwd(i, stream)
        if ev_fwd is not None:
            ev_fwd[1].record(stream)
        if ev_bwd is not None:
            ev_bwd[0].record(stream)
        bwd(i, stream)
        if ev_bwd is not None:
            ev_bwd[1].record(stream)

    for i in range(warmup):
        step(i)
    # the GPU's clocks and power, read while the warm-up steps still run (so the
    # GPU does not idle between the warm-up and the timed region)
    state_before = gpu_state()
    torch.cuda.synchronize()

    # The timed region: K steps, two events per step around the backward (the
    # roofline kernel), recorded on the stream the kernels run on.
    events = [[TimingEvent() for _ in range(2)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i, ev_bwd=events[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    state_after = gpu_state()
    bwd_each = sorted(e[0].elapsed_time(e[1]) for e in events)
    bwd_ms = sum(bwd_each) / steps

    # Outside the timed region: the same steps again with the events around
    # the forward instead, for the per-kernel breakdown.
    fwd_events = [[TimingEvent() for _ in range(2)] for _ in range(steps)]
    for i in range(steps):
        step(i, ev_fwd=fwd_events[i])
    torch.cuda.synchronize()
    fwd_each = sorted(e[0].elapsed_time(e[1]) for e in fwd_events)
    fwd_ms = sum(fwd_each) / steps

    # Also outside it: the same calls captured once into HIP graphs and
    # replayed, the GPU's own time for them.  At the small configurations a
    # call launched from Python costs the host longer than its kernels take,
    # so the eager step above is the host's launch rate there, not the GPU's.
    graph_step_ms = graph_replay_ms(lambda i, st: (fwd(i, st), bwd(i, st)), steps)
    graph_fwd_ms = graph_replay_ms(fwd, steps)
    graph_bwd_ms = graph_replay_ms(bwd, steps)
    # The same replay on one set of tensors: what a step costs when its inputs
    # are still in L2 and the Infinity Cache (a layer whose input the previous
    # op has just written).  Differs from the rotating sets only for the small
    # configurations.
    graph_step_one_set_ms = graph_replay_ms(lambda i, st: (fwd(0, st), bwd(0, st)), steps)

    # What gamma costs the forward: the same calls with gamma == NULL (ag::rms's
    # forward; the same traffic less gamma's per-row loads), replayed likewise.
    def fwd_no_gamma(i, st):
        x, g, dy, y, inv, dx, dg = sets[i % nsets]
        agk.rmsnorm_fwd(x, None, cfg.eps, y=y, inv_rms=inv, stream=st)
    graph_fwd_no_gamma_ms = graph_replay_ms(fwd_no_gamma, steps)

    ms_per_step = wall * 1e3 / steps
    alg = cfg.algorithmic_bytes()
    value = alg / (ms_per_step * 1e-3) / 1e9
    bwd_gbs = cfg.bwd_bytes() / (bwd_ms * 1e-3) / 1e9
    fwd_gbs = cfg.fwd_bytes() / (fwd_ms * 1e-3) / 1e9
    traffic, traffic_src = _traffic(cfg_name)

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg.dtype,
        "data": ("synthetic: x~N(0,%g), gamma~U(0.5,1.5), dy~N(0,1) drawn on the device "
                 "(torch Philox), %d rotating input sets" % (cfg.x_std, nsets)),
        "config": {
            "workload": f"{cfg.name}: RMSNorm layer fwd+VJP x{list(cfg.shape)} {cfg.dtype}, "
                        f"eps {cfg.eps:g}",
            "rows": R,
            "cols": D,
            "algorithmic_bytes_per_step": alg,
            "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
            "rows_per_s": round(R / (ms_per_step * 1e-3), 1),
        },
        "roofline": {
            "kernel": "agk_rmsnorm_bwd (" + _bwd_kernels(agk, R, D, cfg.dtype) + ")",
            "bound": "hbm",
            "achieved": round(bwd_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(bwd_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "algorithmic_bytes_per_launch": cfg.bwd_bytes(),
            "avg_launch_ms": round(bwd_ms, 5),
        },
        "kernels": {
            "fwd": {"avg_ms": round(fwd_ms, 5), "median_ms": round(fwd_each[steps // 2], 5),
                    "alg_bytes": cfg.fwd_bytes(),
                    "gbs": round(fwd_gbs, 2), "frac": round(fwd_gbs / HBM_PEAK_GBS, 4)},
            "bwd": {"avg_ms": round(bwd_ms, 5), "median_ms": round(bwd_each[steps // 2], 5),
                    "alg_bytes": cfg.bwd_bytes(),
                    "gbs": round(bwd_gbs, 2), "frac": round(bwd_gbs / HBM_PEAK_GBS, 4)},
            "gpu_state": {"before_timed": state_before, "after_timed": state_after,
                          "how": "sysfs (hwmon, pp_dpm) of this GPU, read during the last "
                                 "warm-up steps and right after the timed region"},
        },
        "graph": {
            "how": (f"the {steps} steps (then {steps} forwards, then {steps} backwards) "
                    "captured once into a HIP graph and replayed, best of 5 replays: the "
                    "GPU's time without the host's per-call launch cost"),
            "ms_per_step": round(graph_step_ms, 5),
            "gbs": round(alg / (graph_step_ms * 1e-3) / 1e9, 2),
            "pct_of_hbm_peak": round(100.0 * alg / (graph_step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
            "fwd_ms": round(graph_fwd_ms, 5),
            "bwd_ms": round(graph_bwd_ms, 5),
            "ms_per_step_one_set": round(graph_step_one_set_ms, 5),
            "fwd_no_gamma_ms": round(graph_fwd_no_gamma_ms, 5),
            "fwd_gamma_cost_pct": round(100.0 * (graph_fwd_ms / graph_fwd_no_gamma_ms - 1.0), 2),
        },
        "cpu_baseline": None,
    }
    del sets, ws
    torch.cuda.empty_cache()
    if cpu_seconds > 0:
        out["cpu_baseline"] = cpu_baseline(cfg, cpu_seconds)
    return out


def cpu_baseline_c5(sample_rows=256):
    """The CPU oracle of the RMSNorm + linear layer (oracle.rmsnorm_linear_layer:
    the reference's rms_norm(x) * gamma -> matmul W forward and VJP restated,
    bf16 storage, products in float64 through numpy's BLAS) on sample_rows of
    the M = 8192 rows, with the full W [4096, 11008]; median of CPU_RUNS runs.
    Reported as the three products' TFLOP/s, the GPU line's unit."""
    import numpy as np

    import oracle
    _, K, N = C5_SHAPE
    info = host_info()
    rng = np.random.default_rng(0)
    x = oracle.bf16_encode(rng.standard_normal((sample_rows, K), dtype=np.float32))
    g = oracle.bf16_encode(rng.uniform(0.5, 1.5, K).astype(np.float32))
    w = oracle.bf16_encode((rng.standard_normal((K, N), dtype=np.float32) * 0.02))
    dy = oracle.bf16_encode(rng.standard_normal((sample_rows, N), dtype=np.float32))
    oracle.set_threads(info["usable_cpus"])
    _keep_freed_memory()
    oracle.rmsnorm_linear_layer(x, g, w, dy, 1e-5)  # untimed
    times = []
    for _ in range(CPU_RUNS):
        t0 = time.perf_counter()
        oracle.rmsnorm_linear_layer(x, g, w, dy, 1e-5)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    flops = 3 * 2.0 * sample_rows * K * N
    return {"value": round(flops / med / 1e12, 4), "unit": "TFLOP/s",
            "cores": info["usable_cpus"], "kind": "port",
            "sample": (f"{sample_rows} of {C5_SHAPE[0]} rows of x with the full W "
                       f"[{K}, {N}]: the oracle's restatement of the layer's forward + VJP "
                       f"(bf16 storage, float64 products through numpy's BLAS), median of "
                       f"{CPU_RUNS} runs {med:.3f} s"),
            "host": info}


C5_SHAPE = (8192, 4096, 11008)   # x [M, K], W [K, N], dy [M, N]
MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16


def run_c5(steps, warmup, cpu=True):
    """RMSNorm + linear layer (configuration c5): forward + full VJP on one GPU.

    fwd: agk_rmsnorm_fwd (h, inv_rms) -> GEMM y = h W
    bwd: GEMM dW = h^T dy (fp32 result) -> GEMM dh = dy W^T -> agk_rmsnorm_bwd (dx,
         dgamma from dh)
    dW runs before dh: dh then feeds the RMSNorm backward straight from the
    caches, and the step measured about 8 us shorter that way (1725-1729 us
    against 1733-1737 us with dh first).
    Every operand is read in the layout it has (W [K, N], h^T and dy with their k
    strided): the GEMM stages either layout itself, so no transposed copy is made.
    The three products are 3 * 2*M*N*K flops; torch.matmul (hipBLASLt) is timed
    on the same operands in the same run for comparison.
    """
    import torch

    import cgadimpl_amd as agk

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    M, K, N = C5_SHAPE
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    x = torch.randn(M, K, generator=gen, device=dev).bfloat16()
    g = (torch.rand(K, generator=gen, device=dev) + 0.5).bfloat16()
    W = (torch.randn(K, N, generator=gen, device=dev) * 0.02).bfloat16()
    dy = torch.randn(M, N, generator=gen, device=dev).bfloat16()
    eps = 1e-5
    h = torch.empty_like(x)
    inv = torch.empty(M, dtype=torch.float32, device=dev)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    dh = torch.empty_like(x)
    dW = torch.empty(K, N, dtype=torch.float32, device=dev)
    dx = torch.empty_like(x)
    dg = torch.empty(K, dtype=torch.float32, device=dev)
    ws_n = torch.empty(max(1, agk.rmsnorm_bwd_workspace_bytes(M, K)), dtype=torch.uint8, device=dev)

    def gemm_ws(m, n, k, ta, tb):  # the workspace a product asks for (none, on this build)
        need = agk.gemm_bf16_workspace_bytes(m, n, k, ta, tb)
        return torch.empty(need, dtype=torch.uint8, device=dev) if need else None
    ws_y = gemm_ws(M, N, K, False, False)
    ws_dh = gemm_ws(M, K, N, False, True)
    ws_w = gemm_ws(K, N, M, True, False)
    stream = torch.cuda.current_stream()
    stages = ["rmsnorm_fwd", "gemm_y", "gemm_dW", "gemm_dh", "rmsnorm_bwd"]

    def step(ev=None):
        def mark(i):
            if ev is not None:
                ev[i].record(stream)
        mark(0)
        agk.rmsnorm_fwd(x, g, eps, y=h, inv_rms=inv, stream=stream)
        mark(1)
        agk.gemm_bf16(h, W, y, workspace=ws_y, stream=stream)
        mark(2)
        agk.gemm_bf16(h, dy, dW, trans_a=True, workspace=ws_w, stream=stream)
        mark(3)
        agk.gemm_bf16(dy, W, dh, trans_b=True, workspace=ws_dh, stream=stream)
        mark(4)
        agk.rmsnorm_bwd(x, g, inv, dh, dx=dx, dgamma=dg, workspace=ws_n, stream=stream)
        mark(5)

    for _ in range(warmup):
        step()
    state_before = gpu_state()  # read while the warm-up steps still run
    torch.cuda.synchronize()
    events = [[TimingEvent() for _ in range(len(stages) + 1)] for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        step(events[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    state_after = gpu_state()
    per = {name: sum(e[i].elapsed_time(e[i + 1]) for e in events) / steps
           for i, name in enumerate(stages)}

    def lib_ms(f, reps=max(3, steps)):
        for _ in range(2):
            f()
        torch.cuda.synchronize()
        a, b = TimingEvent(), TimingEvent()
        a.record(stream)
        for _ in range(reps):
            f()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    # each product alone, back to back, as hipBLASLt is timed below (the
    # timed step above runs them in the layer's order, between the RMSNorm
    # kernels, which costs a few percent of clock)
    alone_ms = {
        "gemm_y": lib_ms(lambda: agk.gemm_bf16(h, W, y, workspace=ws_y, stream=stream)),
        "gemm_dh": lib_ms(lambda: agk.gemm_bf16(dy, W, dh, trans_b=True, workspace=ws_dh,
                                                stream=stream)),
        "gemm_dW": lib_ms(lambda: agk.gemm_bf16(h, dy, dW, trans_a=True, workspace=ws_w,
                                                stream=stream))}
    # The forward product with the RMSNorm carried into it (normalize-on-load,
    # y = diag(r) (x diag(gamma)) W: kscale = gamma, rowscale = inv_rms) instead
    # of reading the materialised h.  A k-scale runs on the register-staged
    # kernel (the direct-to-LDS kernel has no register stage to apply it in),
    # so this is the price of not writing h.
    g32 = g.float().contiguous()
    kscale_ms = lib_ms(lambda: agk.gemm_bf16(x, W, y, kscale=g32, rowscale=inv, stream=stream))
    torch_ms = {"gemm_y": lib_ms(lambda: h @ W), "gemm_dh": lib_ms(lambda: dy @ W.t()),
                "gemm_dW": lib_ms(lambda: h.t() @ dy)}
    flops = 2.0 * M * N * K
    gemm_ms = per["gemm_y"] + per["gemm_dh"] + per["gemm_dW"]
    tflops = 3 * flops / (gemm_ms * 1e-3) / 1e12
    ms_per_step = wall * 1e3 / steps
    norm_bytes = 5 * M * K * 2 + 2 * K * 2 + 2 * M * 4 + K * 4
    norm_ms = per["rmsnorm_fwd"] + per["rmsnorm_bwd"]
    return {
        "metric": "RMSNorm+linear fwd+VJP (c5): GEMM TFLOP/s on bf16 MFMA (% of 2.5 PF dense)",
        "value": round(tflops, 1),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: x~N(0,1), gamma~U(0.5,1.5), W~N(0,0.02^2), dy~N(0,1) (torch Philox)",
        "config": {"workload": "c5: rms_norm(x) * gamma -> matmul W, fwd + VJP (dx, dgamma, dW)",
                   "M": M, "K": K, "N": N, "gemm_flops_per_step": 3 * flops},
        "roofline": {"kernel": "gemm_nt_direct (3 products)", "bound": "mfma",
                     "achieved": round(tflops, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": None},
        "stages_ms": {k: round(v, 4) for k, v in per.items()},
        "gpu_state": {"before_timed": state_before, "after_timed": state_after},
        "rmsnorm_gbs": round(norm_bytes / (norm_ms * 1e-3) / 1e9, 1),
        "alone_ms": {k: round(v, 4) for k, v in alone_ms.items()},
        "gemm_y_normalize_on_load_ms": round(kscale_ms, 4),
        "torch_hipblaslt_ms": {k: round(v, 4) for k, v in torch_ms.items()},
        "torch_hipblaslt_tflops": round(3 * flops / (sum(torch_ms.values()) * 1e-3) / 1e12, 1),
        "cpu_baseline": cpu_baseline_c5() if cpu else None,
    }


# ---- row ops on the same skeleton (include/agk_rowops.h) ---------------------------
# Algorithmic bytes per kernel launch, s = storage bytes, R rows, D cols:
#   layernorm    fwd 2RDs + 8R (mean, rstd)      bwd 3RDs + 8R
#   softmax      fwd 2RDs                         bwd 3RDs
#   logsumexp    fwd RDs + Rs                     bwd 2RDs + Rs      jvp 2RDs + Rs
#   rmsnorm_jvp  jvp 3RDs + 2Ds + 4R
#   rms_mul      the reference's unfused layer ag::rms(x) * gamma: rms fwd 2RDs + 4R,
#                mul fwd 2RDs + Ds, one-pass bwd (agk_rms_mul_bwd: read x, gy; write
#                dr = gy*gamma and dx; gamma, inv_rms, dgamma) 4RDs + Ds + 4R + 4D
ROWOPS = ("layernorm", "softmax", "logsumexp", "rmsnorm_jvp", "rms_mul")


def _rowop_bytes(op, R, D, s):
    rd = R * D * s
    return {
        "layernorm": {"fwd": 2 * rd + 8 * R, "bwd": 3 * rd + 8 * R},
        "softmax": {"fwd": 2 * rd, "bwd": 3 * rd},
        "logsumexp": {"fwd": rd + R * s, "bwd": 2 * rd + R * s, "jvp": 2 * rd + R * s},
        "rmsnorm_jvp": {"jvp": 3 * rd + 2 * D * s + 4 * R},
        "rms_mul": {"rms": 2 * rd + 4 * R, "mul": 2 * rd + D * s,
                    "bwd": 4 * rd + D * s + 4 * R + 4 * D},
    }[op]


def _oracle_rms_mul(x, g, dy, eps):
    """The oracle's restatement of rms(x) * gamma forward and both VJPs (the
    C oracle with gamma applied, as the reference composes them)."""
    import oracle
    _, inv = oracle.fwd(x, g, eps)
    oracle.bwd(x, g, inv, dy)


def _rowop_cpu_baseline(op, cfg, seconds):
    """The oracle's restatement of the reference rule (numpy, materialising every
    intermediate) on a bounded row sample, timed on this host."""
    import numpy as np

    from cgadimpl_amd import configs
    from oracle import rowops as ro
    rows = max(1, min(cfg.rows, (1 << 20) // cfg.cols))
    x, g, dy = configs.config_inputs(cfg, (rows, cfg.cols))
    if cfg.dtype == "bf16":
        import oracle
        x, g, dy = oracle.bf16_decode(x), oracle.bf16_decode(g), oracle.bf16_decode(dy)
    fns = {
        "layernorm": lambda: ro.layernorm_bwd(x, *ro.layernorm_fwd(x, cfg.eps)[1:], dy, cfg.eps),
        "softmax": lambda: ro.softmax_bwd(ro.softmax_fwd(x), dy),
        "logsumexp": lambda: (ro.logsumexp_fwd(x), ro.logsumexp_bwd(x, dy[:, :1]),
                              ro.logsumexp_jvp(x, dy)),
        "rmsnorm_jvp": lambda: ro.rmsnorm_jvp(x, g, dy, g[::-1] - 1.0, cfg.eps),
        "rms_mul": lambda: _oracle_rms_mul(x, g, dy, cfg.eps),
    }
    f = fns[op]
    f()
    reps, t0 = 0, time.perf_counter()
    while True:
        f()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    alg = sum(_rowop_bytes(op, rows, cfg.cols, cfg.storage_bytes).values())
    return {"value": round(alg * reps / el / 1e9, 3), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"{rows} of {cfg.rows} rows x {cfg.cols} ({cfg.dtype}), the oracle's "
                      f"numpy restatement of the reference rules (fp32, every intermediate "
                      f"materialised), {reps} reps in {el:.1f} s"}


def run_rowop(op, cfg_name, steps, warmup, cpu_seconds):
    import torch

    import cgadimpl_amd as agk
    from cgadimpl_amd import configs

    cfg = configs.CONFIGS[cfg_name]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    R, D = cfg.rows, cfg.cols
    x, g, dy = _device_inputs(cfg, dev, cfg.seed)
    if op in ("softmax", "logsumexp"):
        x = (x * 4.0).contiguous()
    f32 = torch.float32
    out = torch.empty_like(x)
    y = torch.empty_like(x)
    mean = torch.empty(R, 1, dtype=f32, device=dev)
    rstd = torch.empty(R, 1, dtype=f32, device=dev)
    lse = torch.empty(R, 1, dtype=x.dtype, device=dev)
    tl = torch.empty(R, 1, dtype=x.dtype, device=dev)
    dl = dy[:, :1].contiguous()
    tg = (torch.flip(g, [0]) - 1.0).contiguous()
    _, inv = agk.rmsnorm_fwd(x, g, cfg.eps)
    inv1 = torch.empty(R, dtype=f32, device=dev)
    dxo = torch.empty_like(x)
    dgo = torch.empty(D, dtype=f32, device=dev)
    dro = torch.empty_like(x) if op == "rms_mul" else None
    wso = (torch.empty(max(1, agk.rmsnorm_bwd_workspace_bytes(R, D)), dtype=torch.uint8,
                       device=dev) if op == "rms_mul" else None)
    stream = torch.cuda.current_stream()
    launches = {
        "layernorm": [("fwd", lambda: agk.layernorm_fwd(x, cfg.eps, y=y, mean=mean, rstd=rstd,
                                                        stream=stream)),
                      ("bwd", lambda: agk.layernorm_bwd(x, mean, rstd, dy, dx=out,
                                                        stream=stream))],
        "softmax": [("fwd", lambda: agk.softmax_fwd(x, y=y, stream=stream)),
                    ("bwd", lambda: agk.softmax_bwd(y, dy, dz=out, stream=stream))],
        "logsumexp": [("fwd", lambda: agk.logsumexp_fwd(x, y=lse, stream=stream)),
                      ("bwd", lambda: agk.logsumexp_bwd(x, dl, dz=out, stream=stream)),
                      ("jvp", lambda: agk.logsumexp_jvp(x, dy, ty=tl, stream=stream))],
        "rmsnorm_jvp": [("jvp", lambda: agk.rmsnorm_jvp(x, g, inv, dy, tg, ty=out,
                                                        stream=stream))],
        "rms_mul": [("rms", lambda: agk.rmsnorm_fwd(x, None, cfg.eps, y=y, inv_rms=inv1,
                                                    stream=stream)),
                    ("mul", lambda: agk.mul_rowbcast_fwd(y, g, y=out, stream=stream)),
                    ("bwd", lambda: agk.rms_mul_bwd(x, g, inv1, dy, dx=dxo, dgamma=dgo,
                                                    dr=dro, workspace=wso, stream=stream))],
    }[op]
    for _ in range(warmup):
        for _, f in launches:
            f()
    torch.cuda.synchronize()
    n = len(launches)
    ev = [[TimingEvent() for _ in range(n + 1)] for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        ev[i][0].record(stream)
        for k, (_, f) in enumerate(launches):
            f()
            ev[i][k + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    alg = _rowop_bytes(op, R, D, cfg.storage_bytes)
    kernels = {}
    for k, (name, _) in enumerate(launches):
        ms = sum(e[k].elapsed_time(e[k + 1]) for e in ev) / steps
        gbs = alg[name] / (ms * 1e-3) / 1e9
        kernels[name] = {"avg_ms": round(ms, 5), "alg_bytes": alg[name], "gbs": round(gbs, 1),
                         "frac": round(gbs / HBM_PEAK_GBS, 4)}
    dom = max(kernels, key=lambda k: kernels[k]["alg_bytes"])
    ms_per_step = wall * 1e3 / steps
    total = sum(alg.values())
    rec = {
        "metric": f"{op} ({'+'.join(alg)}) achieved HBM GB/s at {list(cfg.shape)}",
        "value": round(total / (ms_per_step * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": cfg.dtype,
        "data": "synthetic: inputs drawn on the device (torch Philox) with the configuration's "
                "distributions" + (" (x scaled by 4 as logits)" if op in ("softmax", "logsumexp")
                                   else ""),
        "config": {"workload": f"{cfg.name}: {op} x{list(cfg.shape)} {cfg.dtype}", "rows": R,
                   "cols": D, "algorithmic_bytes_per_step": total},
        "roofline": {"kernel": {"rmsnorm_jvp": "agk_rmsnorm_jvp",
                                "rms_mul": "agk_rms_mul_bwd"}.get(op, f"agk_{op}_{dom}"),
                     "bound": "hbm", "achieved": kernels[dom]["gbs"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": kernels[dom]["frac"], "traffic": None,
                     "algorithmic_bytes_per_launch": alg[dom],
                     "avg_launch_ms": kernels[dom]["avg_ms"]},
        "kernels": kernels,
        "cpu_baseline": _rowop_cpu_baseline(op, cfg, cpu_seconds) if cpu_seconds > 0 else None,
    }
    return rec


def copy_probe(mib, steps):
    """Device-to-device copies of a known size (torch's copy kernel).

    Under rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE this gives the counter's
    reading for exactly mib MiB read and mib MiB written per dispatch, the
    factor that turns the counters into HBM bytes for the RMSNorm kernels.
    """
    import torch
    n = (mib << 20) // 4
    src = torch.randn(n, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_each_way": n * 4, "dispatches": steps}), flush=True)


STREAM_MIXES = (("copy (1 read + 1 write, as the forward)", 1, 1),
                ("2 reads + 1 write (as the backward)", 2, 1),
                ("2 reads + 2 writes (as the rms(x) * gamma backward)", 2, 2),
                ("read only", 1, 0))
STREAM_GRIDS = (0, 1024, 8192, 65536)  # 0: one workgroup per 16 KiB chunk


def stream_probe(mib, steps):
    """The practical HBM ceiling of this device for the path's traffic mixes.

    A streaming kernel (agk_probe_stream in libagk_bench.so: 16-byte slots, four in flight per
    lane) over MIB-MiB buffers, with plain and with non-temporal accesses, one
    workgroup per 16 KiB chunk (grid 0, how the row kernels touch memory) and
    grid-stride at several grid sizes; HIP events on the launch stream.
    Prints one JSON line per (mix, cache policy) with each grid's GB/s and the
    best.
    """
    import torch

    import cgadimpl_amd as agk
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    nbytes = mib << 20
    a = torch.randint(0, 1 << 30, (nbytes // 4,), dtype=torch.int32, device=dev)
    b = torch.randint(0, 1 << 30, (nbytes // 4,), dtype=torch.int32, device=dev)
    c = torch.empty_like(a)
    d = torch.empty_like(a)
    stream = torch.cuda.current_stream()
    results = []
    for name, reads, writes in STREAM_MIXES:
        for nt in (False, True):
            per_grid = {}
            for grid in STREAM_GRIDS:
                def launch():
                    probe_stream(a, b, c, d, nbytes, reads, writes, nt, grid, stream)
                for _ in range(3):
                    launch()
                e0, e1 = TimingEvent(), TimingEvent()
                e0.record(stream)
                for _ in range(steps):
                    launch()
                e1.record(stream)
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / steps
                per_grid[grid] = round((reads + writes) * nbytes / (us * 1e-6) / 1e9, 1)
            best = max(per_grid.values())
            rec = {"stream_probe": name, "reads": reads, "writes": writes, "nontemporal": nt,
                   "mib_per_buffer": mib, "launches": steps, "gbs_by_grid": per_grid,
                   "best_gbs": best, "pct_of_hbm_peak": round(100.0 * best / HBM_PEAK_GBS, 2)}
            results.append(rec)
            print(json.dumps(rec), flush=True)
    return results


def mfma_probe(reps):
    """What the matrix cores sustain on this device: the bf16 GEMM's inner loop
    without its global loads and barriers (agk_probe_mfma in libagk_bench.so),
    256 workgroups of 4 waves (one wave per SIMD, as the GEMM), each wave 16
    v_mfma_f32_32x32x16_bf16 accumulators.  Mode "lds": the GEMM's fragment
    reads from LDS one substep ahead of the MFMAs; mode "registers": MFMAs
    only; modes "lds, 16x16x32" and "registers, 16x16x32": the same on
    v_mfma_f32_16x16x32_bf16 (8 x 8 accumulators of 16 x 16 per wave, 128
    MFMAs per k-step).  Operand contents: the c5 products' distributions (A ~ N(0,1),
    B ~ N(0,0.02^2) in bf16), uniform +-[0.5, 2), and zeros.  HIP events give
    TFLOP/s; wave 0 of every workgroup reads s_memtime and s_memrealtime
    (100 MHz) around its loop, which give the shader clock it ran at and its
    cycles per 64-deep k-step (64 MFMAs: 2048 cycles at the full rate).  One
    JSON line per (mode, data)."""
    import ctypes

    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = _bench_lib()
    wg, ksteps = 256, 20000
    flop = wg * 4 * ksteps * 64 * 32768
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    half = 256 * 64  # bf16 per operand half of the 64 KiB tile

    def uniform_pm():
        mag = torch.rand(2 * half, generator=gen, device=dev) * 1.5 + 0.5
        sign = torch.randint(0, 2, (2 * half,), generator=gen, device=dev) * 2 - 1
        return (mag * sign).bfloat16()
    datas = (
        ("c5 operands (A ~ N(0,1), B ~ N(0,0.02^2))",
         torch.cat([torch.randn(half, generator=gen, device=dev),
                    torch.randn(half, generator=gen, device=dev) * 0.02]).bfloat16()),
        ("uniform +-[0.5, 2)", uniform_pm()),
        ("zeros", torch.zeros(2 * half, dtype=torch.bfloat16, device=dev)),
    )
    out = torch.empty(wg * 4, dtype=torch.float32, device=dev)
    clocks = torch.zeros(wg * 4, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream()
    recs = []
    for mode, mode_name in ((0, "lds"), (1, "registers"), (2, "lds, 16x16x32"),
                            (3, "registers, 16x16x32")):
        for name, src in datas:
            src = src.contiguous()

            def launch(ck=None):
                rc = lib.agk_probe_mfma(src.data_ptr(), out.data_ptr(),
                                        ck.data_ptr() if ck is not None else None, wg, ksteps,
                                        mode, stream.cuda_stream)
                if rc != 0:
                    raise RuntimeError(f"agk_probe_mfma failed ({rc})")
            for _ in range(2):
                launch()
            e0, e1 = TimingEvent(), TimingEvent()
            e0.record(stream)
            for _ in range(reps):
                launch()
            e1.record(stream)
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / reps
            launch(clocks)
            torch.cuda.synchronize()
            c = clocks.view(wg, 4).cpu().double()
            shader = c[:, 1] - c[:, 0]
            real = c[:, 3] - c[:, 2]
            ghz = (shader / real * 0.1).median().item()
            cyc = (shader / ksteps).median().item()
            tflops = flop / (ms * 1e-3) / 1e12
            rec = {"mfma_probe": mode_name, "data": name, "workgroups": wg,
                   "k_steps_per_wave": ksteps, "launches": reps, "ms_per_launch": round(ms, 3),
                   "tflops": round(tflops, 1),
                   "pct_of_dense_peak": round(100.0 * tflops / MFMA_BF16_PEAK_TFLOPS, 1),
                   "shader_ghz": round(ghz, 3), "cycles_per_k_step": round(cyc, 1),
                   "ideal_cycles_per_k_step": 2048}
            recs.append(rec)
            print(json.dumps(rec), flush=True)
    return recs


def gemm_f32_bench(reps):
    """The graph layer's fp32 matmul (agk_gemm_f32, the fp32 MFMA kernel) at
    square and layer-like sizes in its four layouts, against torch's fp32
    matmul (the vendor library) on the same operands; HIP events on the
    launch stream, after warm-up calls.  One JSON line per shape."""
    import torch

    import cgadimpl_amd as agk
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)

    def ms_of(f):
        for _ in range(3):
            f()
        torch.cuda.synchronize()
        e0, e1 = TimingEvent(), TimingEvent()
        e0.record(stream)
        for _ in range(reps):
            f()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps
    recs = []
    for M, N, K in ((4096, 4096, 4096), (8192, 4096, 4096), (1024, 1024, 1024)):
        rec = {"gemm_f32": f"{M}x{N}x{K}", "tflops": {}, "torch_tflops": {}}
        for ta in (False, True):
            for tb in (False, True):
                a = torch.randn((K, M) if ta else (M, K), generator=gen, device=dev)
                b = torch.randn((N, K) if tb else (K, N), generator=gen, device=dev)
                c = torch.empty(M, N, device=dev)
                tag = ("At" if ta else "A") + ("Bt" if tb else "B")
                ms = ms_of(lambda: agk.gemm_f32(a, b, c=c, trans_a=ta, trans_b=tb,
                                                stream=stream))
                at, bt = (a.t() if ta else a), (b.t() if tb else b)
                tms = ms_of(lambda: torch.matmul(at, bt, out=c))
                rec["tflops"][tag] = round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1)
                rec["torch_tflops"][tag] = round(2.0 * M * N * K / (tms * 1e-3) / 1e12, 1)
                del a, b, c
        rec["pct_of_fp32_matrix_peak"] = round(100.0 * max(rec["tflops"].values()) / 157.3, 1)
        recs.append(rec)
        print(json.dumps(rec), flush=True)
    return recs


WIDE_SHAPES = (("f32", 8, 262144), ("f32", 1, 1 << 20), ("f32", 51, 32768),
               ("f32", 256, 65536), ("f32", 4096, 32768), ("bf16", 8, 262144),
               ("bf16", 51, 32768), ("bf16", 1024, 65536), ("bf16", 16384, 20480),
               ("f32", 2048, 65536), ("bf16", 8192, 131072), ("f32", 2048, 131072),
               ("f32", 256, 262144))


def run_wide(steps):
    """Rows wider than the register-resident kernels: the wide paths against
    the one-workgroup-per-row kernels on the same build, each call captured
    `steps` times into a HIP graph and replayed (GPU time per call).

    forward: out of place (split when the row is too wide for registers),
    the same with a workspace (agk_rmsnorm_fwd_ws: the team kernel where it
    applies, x read once) and in place (y = x, which keeps one workgroup per
    row); backward (dx
    and dgamma) and dx alone as the library takes them with a workspace (the
    one-pass or team kernel where they apply), the same with the team kernel
    switched off (the split path), and dx alone without a workspace
    (looped).  One JSON line per shape; GB/s are algorithmic bytes (forward 2
    tensors, backward 3) over the time.
    """
    import torch

    import cgadimpl_amd as agk
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    out = []
    for dtype, rows, cols in WIDE_SHAPES:
        dt = agk.AGK_F32 if dtype == "f32" else agk.AGK_BF16
        gen = torch.Generator(device=dev)
        gen.manual_seed(rows * 31 + cols)
        tdt = torch.float32 if dtype == "f32" else torch.bfloat16
        x = torch.randn(rows, cols, generator=gen, device=dev).to(tdt)
        g = (torch.rand(cols, generator=gen, device=dev) + 0.5).to(tdt)
        dy = torch.randn(rows, cols, generator=gen, device=dev).to(tdt)
        y, dx = torch.empty_like(x), torch.empty_like(x)
        xin = x.clone()
        inv = torch.empty(rows, dtype=torch.float32, device=dev)
        dg = torch.empty(cols, dtype=torch.float32, device=dev)
        ws = torch.empty(agk.rmsnorm_bwd_workspace_bytes(rows, cols), dtype=torch.uint8,
                         device=dev)
        fws = torch.empty(max(agk.rmsnorm_fwd_workspace_bytes(rows, cols), 8), dtype=torch.uint8,
                          device=dev)
        agk.rmsnorm_fwd(x, g, 1e-6, y=y, inv_rms=inv)
        fn = agk.lib().agk_rmsnorm_bwd

        def dx_only(workspace):
            def body(i, st):
                rc = fn(x.data_ptr(), g.data_ptr(), inv.data_ptr(), dy.data_ptr(), dx.data_ptr(),
                        None, workspace.data_ptr() if workspace is not None else None,
                        workspace.numel() if workspace is not None else 0, rows, cols, dt, 0,
                        st.cuda_stream)
                if rc:
                    raise agk.AgkError(rc, "agk_rmsnorm_bwd")
            return body
        n = max(1, steps)

        def bwd_full(i, st):
            agk.rmsnorm_bwd(x, g, inv, dy, dx=dx, dgamma=dg, workspace=ws, stream=st)
        t = {
            "fwd_split": graph_replay_ms(
                lambda i, st: agk.rmsnorm_fwd(x, g, 1e-6, y=y, inv_rms=inv, stream=st), n),
            "fwd_ws": graph_replay_ms(
                lambda i, st: agk.rmsnorm_fwd(x, g, 1e-6, y=y, inv_rms=inv, workspace=fws,
                                              stream=st), n),
            "fwd_in_place": graph_replay_ms(
                lambda i, st: agk.rmsnorm_fwd(xin, g, 1e-6, y=xin, inv_rms=inv, stream=st), n),
            "bwd": graph_replay_ms(bwd_full, n),
            "bwd_dx": graph_replay_ms(dx_only(ws), n),
        }
        # the same calls with the team kernel switched off (the split path)
        prev = agk.set_team_backward(0)
        try:
            t["bwd_split"] = graph_replay_ms(bwd_full, n)
            t["bwd_dx_split"] = graph_replay_ms(dx_only(ws), n)
        finally:
            agk.set_team_backward(prev)
        t["bwd_dx_looped"] = graph_replay_ms(dx_only(None), n)
        es = x.element_size()
        fb, bb = 2.0 * rows * cols * es, 3.0 * rows * cols * es
        fp, bp = agk.launch_plan(rows, cols, dt, False), agk.launch_plan(rows, cols, dt, True)
        fwp = agk.launch_plan(rows, cols, dt, False, fwd_workspace=True)
        rec = {"wide_rows": f"{dtype} {rows}x{cols}", "dtype": dtype, "rows": rows,
               "cols": cols, "calls_per_graph": n,
               "fwd_plan": fp, "fwd_ws_plan": fwp, "bwd_plan": bp,
               "us": {k: round(v * 1e3, 2) for k, v in t.items()},
               "gbs": {k: round((fb if k.startswith("fwd") else bb) / (v * 1e-3) / 1e9, 1)
                       for k, v in t.items()}}
        print(json.dumps(rec), flush=True)
        out.append(rec)
        del x, g, dy, y, dx, xin, inv, dg, ws, fws
        torch.cuda.empty_cache()
    return out


WIDE_CALLS = ("fwd_split", "fwd_team", "bwd_team", "bwd_split")


def run_wide_call(spec, reps=3):
    """One RMSNorm call on rows wider than the register-resident kernels,
    repeated `reps` times eagerly, for HBM counters (rocprofv3 --pmc): spec is
    DTYPE:ROWS:COLS:CALL with CALL one of WIDE_CALLS -- agk_rmsnorm_fwd (the
    split path), agk_rmsnorm_fwd_ws (the team forward), agk_rmsnorm_bwd with
    the team kernel or with it switched off (the split path).  The inputs and
    the backward's inv_rms are made with torch, so the library's kernels in
    the run are the call's alone.  Prints one JSON line with the call's
    algorithmic bytes."""
    import torch

    import cgadimpl_amd as agk
    dtype, rows, cols, call = spec.split(":")
    rows, cols = int(rows), int(cols)
    if call not in WIDE_CALLS:
        raise SystemExit(f"--wide-call: CALL must be one of {WIDE_CALLS}")
    dev = torch.device("cuda:0")
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    gen = torch.Generator(device=dev)
    gen.manual_seed(rows + cols)
    x = torch.randn(rows, cols, generator=gen, device=dev).to(tdt)
    g = (torch.rand(cols, generator=gen, device=dev) + 0.5).to(tdt)
    dy = torch.randn(rows, cols, generator=gen, device=dev).to(tdt)
    inv = torch.rsqrt(x.float().pow(2).mean(dim=1) + 1e-6).contiguous()
    y, dx = torch.empty_like(x), torch.empty_like(x)
    dg = torch.empty(cols, dtype=torch.float32, device=dev)
    fws = torch.empty(max(agk.rmsnorm_fwd_workspace_bytes(rows, cols), 8), dtype=torch.uint8,
                      device=dev)
    ws = torch.empty(agk.rmsnorm_bwd_workspace_bytes(rows, cols), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    prev = agk.set_team_backward(0 if call == "bwd_split" else 1)
    try:
        for _ in range(reps):
            if call == "fwd_split":
                agk.rmsnorm_fwd(x, g, 1e-6, y=y, inv_rms=inv)
            elif call == "fwd_team":
                agk.rmsnorm_fwd(x, g, 1e-6, y=y, inv_rms=inv, workspace=fws)
            else:
                agk.rmsnorm_bwd(x, g, inv, dy, dx=dx, dgamma=dg, workspace=ws)
            torch.cuda.synchronize()
    finally:
        agk.set_team_backward(prev)
    s = x.element_size()
    n = rows * cols
    alg = (2 * n * s + cols * s + rows * 4 if call.startswith("fwd")
           else 3 * n * s + cols * s + rows * 4 + cols * 4)
    print(json.dumps({"wide_call": call, "dtype": dtype, "rows": rows, "cols": cols,
                      "reps": reps, "algorithmic_bytes": alg}), flush=True)


WIDE_ROWOP_CALLS = ("softmax_fwd", "softmax_bwd", "logsumexp_bwd")


def run_wide_rowop_call(spec, reps=3):
    """One vocabulary-width row-op call repeated `reps` times eagerly, for HBM
    counters: spec is DTYPE:ROWS:COLS:OP:WS with OP one of WIDE_ROWOP_CALLS and
    WS "ws" (the *_ws entry point given a workspace: the team kernel) or "nows"
    (the workspace-free kernel).  Inputs made with torch.  Prints one JSON line
    with the call's algorithmic bytes."""
    import torch

    import cgadimpl_amd as agk
    dtype, rows, cols, op, wsmode = spec.split(":")
    rows, cols = int(rows), int(cols)
    if op not in WIDE_ROWOP_CALLS or wsmode not in ("ws", "nows"):
        raise SystemExit(f"--wide-rowop-call: OP in {WIDE_ROWOP_CALLS}, WS ws or nows")
    dev = torch.device("cuda:0")
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    gen = torch.Generator(device=dev)
    gen.manual_seed(rows + cols)
    z = (torch.randn(rows, cols, generator=gen, device=dev) * 4).to(tdt)
    dy = torch.randn(rows, cols, generator=gen, device=dev).to(tdt)
    dl = torch.randn(rows, 1, generator=gen, device=dev).to(tdt)
    y = torch.softmax(z.float(), dim=-1).to(tdt)
    out = torch.empty_like(z)
    ws = (torch.empty(max(agk.rowops_workspace_bytes(rows, cols), 8), dtype=torch.uint8,
                      device=dev) if wsmode == "ws" else False)
    torch.cuda.synchronize()
    for _ in range(reps):
        if op == "softmax_fwd":
            agk.softmax_fwd(z, y=out, workspace=ws)
        elif op == "softmax_bwd":
            agk.softmax_bwd(y, dy, dz=out, workspace=ws)
        else:
            agk.logsumexp_bwd(z, dl, dz=out, workspace=ws)
        torch.cuda.synchronize()
    n, s = rows * cols, z.element_size()
    alg = {"softmax_fwd": 2 * n * s, "softmax_bwd": 3 * n * s,
           "logsumexp_bwd": 2 * n * s + rows * s}[op]
    print(json.dumps({"wide_call": f"{op} {wsmode}", "dtype": dtype, "rows": rows,
                      "cols": cols, "reps": reps, "algorithmic_bytes": alg}), flush=True)


WIDE_ROWOP_SHAPES = (("bf16", 8192, 128256), ("f32", 8192, 128256), ("bf16", 4096, 151936),
                     ("bf16", 16, 128256), ("bf16", 8192, 50257), ("f32", 8192, 50257),
                     ("bf16", 8192, 65536), ("bf16", 8192, 48000))


def run_wide_rowops(steps):
    """Softmax and log-sum-exp over vocabulary-wide rows (past the resident
    shapes, or not whole 16-byte slots), graph-replayed, on the same values in
    three layouts: 16-byte aligned tensors ("vec"); every tensor one element
    off a 16-byte boundary ("offset": the head/body/tail form of the 16-byte
    looped kernel); the inputs one element off and the outputs aligned
    ("scalar": the element-wise looped kernel; log-sum-exp forward has no row
    output, so it has no such layout).  GB/s are algorithmic bytes: softmax
    forward 2 tensors, backward 3, log-sum-exp forward 1, backward 2."""
    import torch

    import cgadimpl_amd as agk
    dev = torch.device("cuda:0")
    out = []
    for dtype, rows, cols in WIDE_ROWOP_SHAPES:
        tdt = torch.float32 if dtype == "f32" else torch.bfloat16
        gen = torch.Generator(device=dev)
        gen.manual_seed(rows + cols)

        def tensors(shift_in, shift_out):
            def make(vals, shift):
                buf = torch.empty(rows * cols + 8, dtype=tdt, device=dev)
                v = buf[shift:shift + rows * cols].view(rows, cols)
                v.copy_(vals)
                return v
            z = make((torch.randn(rows, cols, generator=gen, device=dev) * 4).to(tdt), shift_in)
            dy = make(torch.randn(rows, cols, generator=gen, device=dev).to(tdt), shift_in)
            zero = torch.zeros(rows, cols, dtype=tdt, device=dev)
            y, dz = make(zero, shift_out), make(zero, shift_out)
            lse = torch.empty(rows, 1, dtype=tdt, device=dev)
            dl = torch.randn(rows, 1, generator=gen, device=dev).to(tdt)
            return z, dy, y, dz, lse, dl

        n = max(1, steps)
        rec = {"wide_rowops": f"{dtype} {rows}x{cols}", "dtype": dtype, "rows": rows,
               "cols": cols, "calls_per_graph": n, "us": {}, "gbs": {},
               "team": {name: {op: agk.rowops_team_plan(op, rows, cols,
                                                        0 if dtype == "f32" else 1, lay)
                               for op in agk.ROWOPS_TEAM_OPS}
                        for name, lay in (("aligned", True), ("offset", False))}}
        es = 4 if dtype == "f32" else 2
        tb = rows * cols * es
        wsb = agk.rowops_workspace_bytes(rows, cols)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev) if wsb else False
        for tag, shift_in, shift_out in (("vec", 0, 0), ("offset", 1, 1), ("scalar", 1, 0)):
            z, dy, y, dz, lse, dl = tensors(shift_in, shift_out)
            t = {
                "softmax_fwd": (graph_replay_ms(
                    lambda i, st: agk.softmax_fwd(z, y=y, workspace=ws, stream=st), n), 2),
                "softmax_bwd": (graph_replay_ms(
                    # y takes the outputs' layout: the inputs' here
                    lambda i, st: agk.softmax_bwd(z, dy, dz=y, workspace=ws, stream=st), n), 3),
                "logsumexp_bwd": (graph_replay_ms(
                    lambda i, st: agk.logsumexp_bwd(z, dl, dz=dz, workspace=ws, stream=st), n),
                    2),
            }
            if tag != "scalar":  # the same calls without a workspace (no team kernel)
                t["softmax_fwd_nows"] = (graph_replay_ms(
                    lambda i, st: agk.softmax_fwd(z, y=y, workspace=False, stream=st), n), 2)
                t["softmax_bwd_nows"] = (graph_replay_ms(
                    lambda i, st: agk.softmax_bwd(z, dy, dz=y, workspace=False, stream=st), n), 3)
                t["logsumexp_bwd_nows"] = (graph_replay_ms(
                    lambda i, st: agk.logsumexp_bwd(z, dl, dz=dz, workspace=False, stream=st),
                    n), 2)
            # the backward from the forward's fp32 value (one streaming pass)
            l32 = agk.logsumexp_fwd_keep(z)[1]
            t["logsumexp_bwd_from_value"] = (graph_replay_ms(
                lambda i, st: agk.logsumexp_bwd_from_value(z, l32, dl, dz=dz, stream=st), n), 2)
            if tag != "scalar":  # no row output: no element-wise layout
                t["logsumexp_fwd"] = (graph_replay_ms(
                    lambda i, st: agk.logsumexp_fwd(z, y=lse, stream=st), n), 1)
            for k, (ms, passes) in t.items():
                rec["us"][f"{k}_{tag}"] = round(ms * 1e3, 1)
                rec["gbs"][f"{k}_{tag}"] = round(passes * tb / (ms * 1e-3) / 1e9, 1)
            del z, dy, y, dz, lse, dl
            torch.cuda.empty_cache()
        print(json.dumps(rec), flush=True)
        out.append(rec)
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=2000,
                    help="untimed steps first (default 2000, ~1.8 s at c2): right after a "
                         "high-power workload, such as the GEMM tests, the GPU needs a second or "
                         "two of load to return to its steady clocks")
    ap.add_argument("--config", default=DEFAULT_CONFIG,
                    help="c1, c2 (default, the headline), c3, c4a, c4b, c4c, c5 (RMSNorm + "
                         "linear), or 'all'")
    ap.add_argument("--op", default="rmsnorm",
                    help="rmsnorm (default: the layer fwd + VJP), or a row op on the same "
                         "skeleton: " + ", ".join(ROWOPS) + ", or 'rowops' for all four")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="0 disables the CPU baseline; any other value runs it (its sample "
                         "size, at least the host's last-level cache per tensor, fixes its work)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run MIB-MiB device copies (counter calibration), then exit")
    ap.add_argument("--stream-probe", type=int, default=0, metavar="MIB",
                    help="only time the HBM streaming probe (copy, 2 reads + 1 write, read "
                         "only; plain and non-temporal) over MIB-MiB buffers, then exit")
    ap.add_argument("--mfma-probe", action="store_true",
                    help="only run the MFMA probe (the bf16 GEMM's inner loop without loads or "
                         "barriers, by operand content, with the shader clock it ran at), then "
                         "exit")
    ap.add_argument("--gemm-f32", action="store_true",
                    help="only time the fp32 GEMM (agk_gemm_f32) against torch's fp32 matmul, "
                         "then exit")
    ap.add_argument("--wide-call", metavar="DTYPE:ROWS:COLS:CALL",
                    help="run one wide-row RMSNorm call three times eagerly (for rocprofv3 "
                         "--pmc): CALL is fwd_split, fwd_team, bwd_team or bwd_split; then exit")
    ap.add_argument("--wide-rowop-call", metavar="DTYPE:ROWS:COLS:OP:WS",
                    help="run one vocabulary-width row-op call three times eagerly (for "
                         "rocprofv3 --pmc): OP is softmax_fwd, softmax_bwd or logsumexp_bwd, "
                         "WS is ws (the team kernel) or nows; then exit")
    ap.add_argument("--wide", action="store_true",
                    help="only time rows wider than the register-resident kernels: the split "
                         "paths against the one-workgroup-per-row kernels, and softmax / "
                         "log-sum-exp at vocabulary widths (16-byte against element-wise "
                         "looped kernels), then exit")
    args = ap.parse_args()
    if args.copy_probe:
        copy_probe(args.copy_probe, args.steps)
        return
    if args.stream_probe:
        stream_probe(args.stream_probe, min(args.steps, 50))
        return
    if args.mfma_probe:
        mfma_probe(min(args.steps, 5))
        return
    if args.gemm_f32:
        gemm_f32_bench(min(args.steps, 10))
        return
    if args.wide_call:
        run_wide_call(args.wide_call)
        return
    if args.wide_rowop_call:
        run_wide_rowop_call(args.wide_rowop_call)
        return
    if args.wide:
        run_wide(min(args.steps, 20))
        run_wide_rowops(min(args.steps, 10))
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        rank = int(os.environ.get("RANK", "0"))
        if rank == 0:
            print(f"bench.py: this build runs the RMSNorm path on one GPU; --gpus {args.gpus} "
                  f"(WORLD_SIZE {world}) is not supported. Rows shard across GPUs with no "
                  "communication except one dgamma reduction, in rank order.", file=sys.stderr)
        sys.exit(2)

    from cgadimpl_amd import configs
    if args.op != "rmsnorm":
        ops = ROWOPS if args.op == "rowops" else [args.op]
        names = ["c2", "c3"] if args.config == "all" else [args.config]
        for name in names:
            for op in ops:
                print(json.dumps(run_rowop(op, name, args.steps, args.warmup,
                                           min(args.cpu_seconds, 5.0))), flush=True)
        return
    names = list(configs.CONFIGS) + ["c5"] if args.config == "all" else [args.config]
    for name in names:
        if name == "c5":
            rec = run_c5(args.steps, args.warmup, cpu=args.cpu_seconds > 0)
        else:
            rec = run(name, args.steps, args.warmup, args.cpu_seconds)
        print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()

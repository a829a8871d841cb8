"""The C++ graph layer (ag::Value, rms, rms_norm, mul, matmul, laynor, softmax_row,
logsumexp_row, backward, jvp, GraphRunner) over the C ABI.

CPU: libag.so and the test program resolve every dependency and export the
reference's API surface.  GPU: the program's self-checks (numerical gradients
in the reference's pattern, accumulation, zero_grad, parallel == sequential
backward, tied gamma, errors, bf16, streams, the row ops' numerical gradients,
forward mode against central differences, matmul against a host fp64
product, hipGraph capture and replay against eager runs) and, through its dump mode, the
fused layer, the fused layer with parallel backward and the unfused graph
rms(x) * gamma against the CPU oracle on seeded inputs.
"""
import os
import subprocess
import tempfile

import numpy as np
import pytest

import oracle
from cgadimpl_amd import LIB_DIR, configs
from gpu_util import as_f32
from tolerances import TOL_BF16, TOL_F32, dx_rel_err, row_rel_err, vec_rel_err

PROGRAM = os.path.join(LIB_DIR, "test_ag_layer")
LIBAG = os.path.join(LIB_DIR, "libag.so")
LAYER_BENCH = os.path.join(LIB_DIR, "rmsnorm_layer")


def test_graph_layer_links_and_exports():
    for path in (PROGRAM, LIBAG, LAYER_BENCH):
        assert os.path.exists(path), "build first: python -c 'import __graft_entry__ as g; g.build()'"
        ldd = subprocess.run(["ldd", path], capture_output=True, text=True, check=True).stdout
        assert "not found" not in ldd, ldd
        assert "libagk_rmsnorm.so" in ldd
    syms = subprocess.run(["nm", "-DC", "--defined-only", LIBAG], capture_output=True, text=True,
                          check=True).stdout
    for want in ("ag::rms(ag::Value const&)", "ag::rms_norm(ag::Value const&, ag::Value const&, float)",
                 "ag::mul(ag::Value const&, ag::Value const&)",
                 "ag::backward(ag::Value const&, ag::Tensor const*, bool)",
                 "ag::zero_grad(ag::Value const&)", "ag::vjp_lookup(ag::Op)",
                 "ag::detail::vjp_RMSNorm(ag::Node*, ag::Tensor const&)",
                 "ag::detail::vjp_Mul(ag::Node*, ag::Tensor const&)",
                 "ag::topo_from(ag::Node*)", "ag::nn::RMSNorm::RMSNorm(long, float, ag::Dtype)",
                 "ag::matmul(ag::Value const&, ag::Value const&)", "ag::laynor(ag::Value const&)",
                 "ag::softmax_row(ag::Value const&)", "ag::logsumexp_row(ag::Value const&)",
                 "ag::jvp_lookup(ag::Op)", "ag::detail::vjp_MatMul(ag::Node*, ag::Tensor const&)",
                 "ag::detail::jvp_RMSNorm(ag::Node*, std::function<ag::Tensor const& (ag::Node*)> const&)",
                 "ag::GraphRunner::begin_capture()", "ag::GraphRunner::end_capture()",
                 "ag::GraphRunner::replay()"):
        assert want in syms, want


@pytest.mark.gpu
def test_graph_layer_selftest(cuda):
    proc = subprocess.run([PROGRAM, "selftest"], capture_output=True, text=True, timeout=240)
    print(proc.stdout)
    print(proc.stderr)
    assert proc.returncode == 0, proc.stdout[-3000:] + proc.stderr[-2000:]
    assert "[FAIL]" not in proc.stdout


DUMP_CASES = [("c1", None), ("c2", (2, 512, 4096)), ("c3", (1, 256, 8192)),
              ("c4a", (1, 61, 5120)), ("c4c", None), ("ragged", (37, 1030))]


@pytest.mark.gpu
@pytest.mark.parametrize("name,shape", DUMP_CASES, ids=[c[0] for c in DUMP_CASES])
def test_graph_layer_against_oracle(cuda, name, shape):
    if name == "ragged":
        cfg = configs.CONFIGS["c1"]
        x, g, dy = configs.make_inputs(shape, seed=5)
    else:
        cfg = configs.CONFIGS[name]
        x, g, dy = configs.config_inputs(cfg, shape)
    cols = x.shape[-1]
    rows = x.size // cols
    dt = 1 if cfg.dtype == "bf16" else 0
    store = np.uint16 if dt else np.float32
    eps = cfg.eps
    print(f"graph layer {name} {rows}x{cols} {cfg.dtype}", flush=True)
    with tempfile.TemporaryDirectory() as d:
        with open(os.path.join(d, "meta.txt"), "w") as fh:
            fh.write(f"{rows} {cols} {dt} {eps!r}\n")
        for nm, a in (("x", x), ("gamma", g), ("dy", dy)):
            np.ascontiguousarray(a).tofile(os.path.join(d, nm + ".bin"))
        proc = subprocess.run([PROGRAM, "dump", d], capture_output=True, text=True, timeout=120)
        assert proc.returncode == 0, proc.stdout + proc.stderr

        def load(nm, dtype=store, shape=(rows, cols)):
            return np.fromfile(os.path.join(d, nm + ".bin"), dtype=dtype).reshape(shape)

        tol = TOL_BF16 if dt else TOL_F32
        xs, dys = x.reshape(rows, cols), dy.reshape(rows, cols)
        for tag, e in (("fused", eps), ("fused_par", eps), ("unfused", 1e-5)):
            ry, rinv = oracle.fwd(xs, g, e)
            rdx, rdg = oracle.bwd(xs, g, rinv, dys)
            y, dx = load("y_" + tag), load("dx_" + tag)
            dg = load("dg_" + tag, np.float32, (cols,))
            # the unfused bf16 graph rounds rms(x) to bf16 before the multiply
            # and the rms node's gradient to bf16 before vjp_RMSNorm
            t = tol
            errs = {"y": row_rel_err(as_f32(y), as_f32(ry)),
                    "dx": dx_rel_err(as_f32(dx), as_f32(rdx), as_f32(xs), as_f32(g),
                                     as_f32(dys), e),
                    "dgamma": vec_rel_err(dg, rdg)}
            if tag != "unfused":
                errs["inv_rms"] = vec_rel_err(load("inv_" + tag, np.float32, (rows,)), rinv)
            print(f"  [{tag}] " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
            for k, v in errs.items():
                assert v <= (TOL_F32 if k == "inv_rms" else t), (tag, k, v)
        # scalar literals: rms(x) * 0.75f and -1.5f * rms(x) (eps 1e-5, as ag::rms)
        # against the oracle's rms scaled by s, and its VJP of s * dy
        ones = np.ones(cols, dtype=np.float32)
        for tag, sc in (("scaled_r", 0.75), ("scaled_l", -1.5)):
            xs32 = as_f32(xs)
            ry, rinv = oracle.fwd(xs32, None, 1e-5)
            rdx, _ = oracle.bwd(xs32, None, rinv, as_f32(dys) * np.float32(sc))
            y, dx = load("y_" + tag), load("dx_" + tag)
            errs = {"y": row_rel_err(as_f32(y), as_f32(ry) * np.float32(sc)),
                    "dx": dx_rel_err(as_f32(dx), as_f32(rdx), xs32, ones,
                                     as_f32(dys) * np.float32(sc), 1e-5)}
            print(f"  [{tag}] " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
            for k, v in errs.items():
                assert v <= tol, (tag, k, v)
        # parallel backward of a single node gives the same bits as sequential
        assert np.array_equal(load("dx_fused"), load("dx_fused_par"))
        assert np.array_equal(load("dg_fused", np.float32, (cols,)),
                              load("dg_fused_par", np.float32, (cols,)))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_layer_benchmark_program_runs(cuda, dtype):
    """The RMSNorm layer benchmark through the graph layer (the program the
    reference's empty Benchmark/RMSNormLayer.cpp stands for) runs both the
    fused layer and the unfused rms(x) * gamma graph, eagerly and as replays of
    a captured step, and reports each."""
    import json
    proc = subprocess.run([LAYER_BENCH, "4", "128", "512", "3", "1", dtype, "both"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-2000:]
    lines = [json.loads(ln) for ln in proc.stdout.splitlines() if ln.startswith("{")]
    got = [(ln["path"].split(", ")[1].split()[0], ln["path"].split(", ")[-1]) for ln in lines]
    assert got == [("nn::RMSNorm", "eager"), ("nn::RMSNorm", "captured"),
                   ("ag::rms(x)", "eager"), ("ag::rms(x)", "captured")]
    for ln in lines:
        assert ln["shape"] == [4, 128, 512] and ln["dtype"] == dtype and ln["steps"] == 3
        assert ln["ms_per_step"] > 0 and ln["gbs"] > 0
    bad = subprocess.run([LAYER_BENCH, "4", "128", "512", "0"], capture_output=True, text=True,
                         timeout=60)
    assert bad.returncode == 1 and "usage" in bad.stderr

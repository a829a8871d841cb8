"""Build recipe for the native libraries of cgadimpl_amd.

Outputs (in-tree, git-ignored, shipped with the source tree):
  cgadimpl_amd/lib/libagk_rmsnorm.so   HIP kernels + C ABI (include/agk_rmsnorm.h,
                                       include/agk_rowops.h)
  cgadimpl_amd/lib/libagk_bench.so     bench.py's measurement probes (csrc/agk_bench.h;
                                       not product ABI)
  cgadimpl_amd/lib/libagk_synth.so     seeded synthetic input generator (host)
  cgadimpl_amd/lib/libag.so            the C++ graph layer (ag::Value, rms, rms_norm,
                                       mul, backward) over the C ABI (host C++)
  cgadimpl_amd/lib/test_ag_layer       its GPU test program (tests/cpp/)
  cgadimpl_amd/lib/rmsnorm_layer       the RMSNorm layer benchmark through the graph layer
                                       (cgadimpl_amd/ag/bench/rmsnorm_layer.cpp)

Every HIP translation unit is compiled for gfx950 only, with packed-fp32
instruction generation disabled.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB = os.path.join(PKG, "lib")
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}")
    # Surface real warnings but not the host pass's note about the GPU feature flag.
    lines = [ln for ln in proc.stdout.splitlines()
             if ln.strip() and "packed-fp32-ops" not in ln and "is not a recognized feature" not in ln]
    if lines:
        sys.stderr.write("\n".join(lines) + "\n")


def _atomic_build(out: str, cmd_for: callable) -> None:
    tmp = out + ".tmp"
    _run(cmd_for(tmp))
    os.replace(tmp, out)


def hip_library(name: str, sources: list[str], extra: list[str] | None = None,
                libs: list[str] | None = None) -> str:
    """Compiles each source to an object (in parallel), then links the library."""
    out = os.path.join(LIB, name)
    objdir = os.path.join(LIB, "obj")
    os.makedirs(objdir, exist_ok=True)

    def compile_one(src: str) -> str:
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        _atomic_build(obj, lambda o: [HIPCC, *HIP_FLAGS, f"-I{INCLUDE}", "-c",
                                      os.path.join(CSRC, src), *(extra or []), "-o", o])
        return obj

    with ThreadPoolExecutor(max_workers=len(sources)) as ex:
        objs = list(ex.map(compile_one, sources))
    _atomic_build(out, lambda o: [HIPCC, *HIP_FLAGS, "-shared", *objs, "-o", o, *(libs or [])])
    return out


def host_library(name: str, sources: list[str], compiler: str = "g++") -> str:
    out = os.path.join(LIB, name)
    srcs = [os.path.join(CSRC, s) for s in sources]
    _atomic_build(out, lambda o: [compiler, "-O2", "-fPIC", "-shared", "-std=c++17", *srcs,
                                  "-o", o])
    return out


# The kernel library's sources (every kernel hand-written: it links nothing
# beyond the HIP runtime).
KERNEL_SOURCES = ["rmsnorm.hip", "gemm.hip", "gemm_f32.hip", "rowops.hip", "bcast.hip"]
KERNEL_LIBS: list[str] = []
# The benchmark's own measurement probes (csrc/agk_bench.h): loaded by bench.py
# only, not part of the product ABI.
BENCH_SOURCES = ["probe.hip", "mfma_probe.hip"]

AG_DIR = os.path.join(PKG, "ag")
AG_SOURCES = ["tensor.cpp", "graph.cpp", "ops.cpp", "autodiff.cpp", "nn.cpp", "runtime.cpp"]
# Host C++ against the HIP runtime API (no device code in these files).
HOST_HIP_FLAGS = ["-std=c++17", "-O2", "-fPIC", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
                  f"-I{ROCM}/include", f"-I{os.path.join(AG_DIR, 'include')}", f"-I{INCLUDE}"]
HOST_HIP_LIBS = [f"-L{LIB}", f"-L{ROCM}/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN",
                 f"-Wl,-rpath,{ROCM}/lib"]


def ag_library(cxx: str = "g++", extra: list[str] | None = None) -> str:
    out = os.path.join(LIB, "libag.so")
    srcs = [os.path.join(AG_DIR, "src", s) for s in AG_SOURCES]
    _atomic_build(out, lambda o: [cxx, *HOST_HIP_FLAGS, *(extra or []), "-shared", *srcs, "-o",
                                  o, f"-L{LIB}", "-lagk_rmsnorm", *HOST_HIP_LIBS])
    return out


def ag_program(name: str, source: str, cxx: str = "g++", extra: list[str] | None = None) -> str:
    out = os.path.join(LIB, name)
    _atomic_build(out, lambda o: [cxx, *HOST_HIP_FLAGS, *(extra or []), source, "-o", o,
                                  f"-L{LIB}", "-lag", "-lagk_rmsnorm", *HOST_HIP_LIBS,
                                  "-pthread"])
    return out


SAN_HOST_FLAGS = ["-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=undefined",
                  "-shared-libsan", "-fno-omit-frame-pointer"]


def build_sanitized(out_dir: str, verbose: bool = True) -> list[str]:
    """The kernel library and the input generator with AddressSanitizer and
    UndefinedBehaviorSanitizer on their host code only (every -fsanitize= goes
    behind -Xarch_host: the gfx950 code is built as usual), into out_dir.  The
    process that loads them must preload the shared sanitizer runtime."""
    global LIB
    saved = LIB
    os.makedirs(out_dir, exist_ok=True)
    host = [f for flag in SAN_HOST_FLAGS for f in ("-Xarch_host", flag)]
    try:
        LIB = out_dir
        outs = [hip_library("libagk_rmsnorm.so", KERNEL_SOURCES, extra=[*host, "-g"],
                            libs=KERNEL_LIBS)]
        clang = os.path.join(ROCM, "llvm", "bin", "clang++")
        out = os.path.join(out_dir, "libagk_synth.so")
        _atomic_build(out, lambda o: [clang, *SAN_HOST_FLAGS, "-g", "-O1", "-fPIC", "-shared",
                                      "-std=c++17", os.path.join(CSRC, "synth.cpp"), "-o", o])
        outs.append(out)
        # the graph layer and its programs (host C++ over the HIP runtime API)
        outs.append(ag_library(clang, [*SAN_HOST_FLAGS, "-g"]))
        outs.append(ag_program("test_ag_layer", os.path.join(ROOT, "tests", "cpp",
                                                             "test_ag_layer.cpp"),
                               clang, [*SAN_HOST_FLAGS, "-g"]))
        outs.append(ag_program("rmsnorm_layer", os.path.join(AG_DIR, "bench",
                                                             "rmsnorm_layer.cpp"),
                               clang, [*SAN_HOST_FLAGS, "-g"]))
    finally:
        LIB = saved
    if verbose:
        for o in outs:
            print(f"built {os.path.relpath(o, ROOT)} (host code sanitised)")
    return outs


def build_all(verbose: bool = True) -> list[str]:
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(LIB, exist_ok=True)
    jobs = [
        lambda: hip_library("libagk_rmsnorm.so", KERNEL_SOURCES, libs=KERNEL_LIBS),
        lambda: hip_library("libagk_bench.so", BENCH_SOURCES),
        lambda: host_library("libagk_synth.so", ["synth.cpp"]),
    ]
    with ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        outs = [f.result() for f in [ex.submit(j) for j in jobs]]
    # the graph layer links the kernel library, its programs link both
    outs.append(ag_library())
    outs.append(ag_program("test_ag_layer", os.path.join(ROOT, "tests", "cpp",
                                                         "test_ag_layer.cpp")))
    outs.append(ag_program("rmsnorm_layer", os.path.join(AG_DIR, "bench", "rmsnorm_layer.cpp")))
    if verbose:
        for o in outs:
            print(f"built {os.path.relpath(o, ROOT)}")
    return outs


if __name__ == "__main__":
    build_all()

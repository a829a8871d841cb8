"""Build recipe for the native libraries of cgadimpl_amd.

Outputs (in-tree, git-ignored, shipped with the source tree):
  cgadimpl_amd/lib/libagk_rmsnorm.so   HIP kernels + C ABI (include/agk_rmsnorm.h)
  cgadimpl_amd/lib/libagk_synth.so     seeded synthetic input generator (host)

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


def hip_library(name: str, sources: list[str], extra: list[str] | None = None) -> str:
    out = os.path.join(LIB, name)
    srcs = [os.path.join(CSRC, s) for s in sources]
    _atomic_build(out, lambda o: [HIPCC, *HIP_FLAGS, "-shared", f"-I{INCLUDE}", *srcs,
                                  *(extra or []), "-o", o])
    return out


def host_library(name: str, sources: list[str], compiler: str = "g++") -> str:
    out = os.path.join(LIB, name)
    srcs = [os.path.join(CSRC, s) for s in sources]
    _atomic_build(out, lambda o: [compiler, "-O2", "-fPIC", "-shared", "-std=c++17", *srcs,
                                  "-o", o])
    return out


def build_all(verbose: bool = True) -> list[str]:
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(LIB, exist_ok=True)
    jobs = [
        lambda: hip_library("libagk_rmsnorm.so", ["rmsnorm.hip"]),
        lambda: host_library("libagk_synth.so", ["synth.cpp"]),
    ]
    with ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        outs = [f.result() for f in [ex.submit(j) for j in jobs]]
    if verbose:
        for o in outs:
            print(f"built {os.path.relpath(o, ROOT)}")
    return outs


if __name__ == "__main__":
    build_all()

"""Build recipe for the CPU oracle (test infrastructure only).

  oracle/liboracle_rmsnorm.so        the restatement, built as-is
  oracle/liboracle_rmsnorm_mut<k>.so built on request with -DORACLE_MUTATION=k
                                     (planted mistakes for the pinning tests)

The reference implementation itself cannot be compiled here: every
arithmetic kernel of the path lives in the un-vendored OwnTensor submodule
(`tensor/` is empty) and the project requires CUDA and MLIR, so there is no
oracle/_ref build.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "rmsnorm_oracle.c")
CFLAGS = ["-O2", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
          "-fno-fast-math", "-Wall"]
# ORACLE_SANITIZE=1 builds with AddressSanitizer and UndefinedBehaviorSanitizer
# (ROCm's clang, shared sanitizer runtime, which the process must preload) into
# ORACLE_LIB_DIR; tests/run_sanitized.py runs the CPU test suite that way.
SANITIZE = os.environ.get("ORACLE_SANITIZE") == "1"
SAN_CC = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin", "clang")
SAN_FLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-shared-libsan",
             "-fno-omit-frame-pointer", "-g"]
LIB_DIR = os.environ.get("ORACLE_LIB_DIR", HERE)


def lib_path(mutation: int = 0) -> str:
    name = "liboracle_rmsnorm.so" if mutation == 0 else f"liboracle_rmsnorm_mut{mutation}.so"
    return os.path.join(LIB_DIR, name)


def build(mutation: int = 0, out: str | None = None) -> str:
    out = out or lib_path(mutation)
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    cc = [SAN_CC, *SAN_FLAGS] if SANITIZE else ["gcc"]
    cmd = [*cc, *CFLAGS, f"-DORACLE_MUTATION={mutation}", SRC, "-o", tmp, "-lm"]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        raise RuntimeError("oracle build failed: " + " ".join(cmd))
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build())

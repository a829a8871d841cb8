#!/usr/bin/env python3
"""Runs the CPU test suite against AddressSanitizer + UndefinedBehaviorSanitizer builds.

Builds, with ROCm's clang and the shared sanitizer runtime:
  oracle/_san/                 the CPU oracle (oracle/build.py, ORACLE_SANITIZE=1)
  cgadimpl_amd/lib/san/        libagk_rmsnorm.so (host code sanitised, gfx950 code as
                               usual: every -fsanitize= goes behind -Xarch_host),
                               libagk_synth.so, libag.so and the graph layer's programs
then runs `pytest tests -m "not gpu"` with the runtime preloaded and the bindings
pointed at those builds (AGK_LIB_DIR, ORACLE_LIB_DIR).  That covers the oracle's
arithmetic on every fixture and pin, the C ABI's argument validation (null and
overflowing sizes, short workspaces, bad dtypes), the input generator and the
graph layer's library loading.  No GPU is needed; the GPU tests are not run.

  python tests/run_sanitized.py            # exit status: pytest's
  python tests/run_sanitized.py -k abi     # extra arguments go to pytest
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
SAN_LIB = os.path.join(ROOT, "cgadimpl_amd", "lib", "san")
SAN_ORACLE = os.path.join(ROOT, "oracle", "_san")


def asan_runtime() -> str:
    found = sorted(glob.glob(os.path.join(ROCM, "llvm", "lib", "clang", "*", "lib", "linux",
                                          "libclang_rt.asan-x86_64.so")))
    if not found:
        raise SystemExit("no shared AddressSanitizer runtime under " + ROCM)
    return found[-1]


def main(argv: list[str]) -> int:
    sys.path.insert(0, ROOT)
    from cgadimpl_amd import _build
    _build.build_sanitized(SAN_LIB)
    env = dict(os.environ)
    env.update({
        "ORACLE_SANITIZE": "1",
        "ORACLE_LIB_DIR": SAN_ORACLE,
        "AGK_LIB_DIR": SAN_LIB,
        "LD_PRELOAD": asan_runtime(),
        # Python and torch keep memory until exit: leak reports would be theirs
        "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1:detect_stack_use_after_return=0",
        "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
    })
    build = [sys.executable, "-c", "import sys; sys.path.insert(0, %r); "
             "from oracle import build; print('built', build.build())" % ROOT]
    rc = subprocess.call(build, env=env, cwd=ROOT)
    if rc:
        return rc
    cmd = [sys.executable, "-m", "pytest", os.path.join(ROOT, "tests"), "-m", "not gpu", "-x",
           "-q", "-p", "no:cacheprovider", *argv]
    print("running:", " ".join(cmd), flush=True)
    return subprocess.call(cmd, env=env, cwd=ROOT)


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))

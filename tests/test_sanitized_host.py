"""Host sanitizers (ASan + UBSan) over the CPU-side code: the oracle, and the
library's host code (argument validation, config checks, context set-up,
the C-ABI error paths), each built with clang's sanitizers
(`make -C oracle sanitize`, `python -m neonengine_amd._build --sanitize`; both
run by __graft_entry__.build()).  A child process preloads clang's ASan
runtime and runs the CPU tests of the oracle and of the C-ABI against those
builds; any sanitizer report fails it.  Device code is not instrumented."""
import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_ASAN = os.path.join(ROOT, "oracle", "_asan", "libneon_oracle.so")
LIB_ASAN = os.path.join(ROOT, "neonengine_amd", "_asan", "libneon_gptoss.so")


def asan_runtime():
    found = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return found[-1] if found else None


def test_cpu_suites_under_host_sanitizers():
    rt = asan_runtime()
    if rt is None or not (os.path.exists(ORACLE_ASAN) and os.path.exists(LIB_ASAN)):
        pytest.skip("sanitizer builds or clang's ASan runtime not present (run build())")
    env = dict(os.environ, LD_PRELOAD=rt, NEON_ORACLE_LIB=ORACLE_ASAN, NEON_GPTOSS_LIB=LIB_ASAN,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", OMP_NUM_THREADS="4")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider",
                        "-m", "not gpu", "-k", "not sanitized",
                        os.path.join(ROOT, "tests", "test_oracle.py"),
                        os.path.join(ROOT, "tests", "test_capi_cpu.py")],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    tail = (r.stdout + r.stderr)[-3000:]
    assert "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, tail
    assert r.returncode == 0, tail

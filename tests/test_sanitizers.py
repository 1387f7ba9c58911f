"""Host C++ under AddressSanitizer + UndefinedBehaviorSanitizer: the CPU
suite (C ABI, tokenizer on untrusted tokenizer.json, Local post-processing,
the oracle) run again against the sanitizer builds of libdecide_hip.so's host
code (decide_amd/csrc/Makefile, `sanitize`) and of the oracle
(oracle/Makefile, `sanitize`), with the sanitizer runtime preloaded into the
Python process. Any report aborts the run (halt_on_error, no recovery).
Leak checking is off: the interpreter itself keeps allocations to exit."""
import glob
import os
import shutil
import subprocess
import sys

import pytest

from conftest import ROOT

HIPCC = "/opt/rocm/bin/hipcc"
CLANG = "/opt/rocm/llvm/bin/clang++"


def asan_runtime():
    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


@pytest.mark.skipif(os.environ.get("DN_UNDER_SANITIZER") == "1", reason="already the sanitized run")
def test_cpu_suite_under_asan_ubsan():
    rt = asan_runtime()
    if not (os.path.exists(HIPCC) and os.path.exists(CLANG) and rt and shutil.which("make")):
        pytest.skip("needs ROCm's hipcc / clang++ and the clang ASan runtime")
    csrc, orc = os.path.join(ROOT, "decide_amd", "csrc"), os.path.join(ROOT, "oracle")
    # The .hip objects of the ordinary build are linked in unchanged.
    subprocess.run(["make", "-s", "-C", csrc, "-j8"], check=True)
    subprocess.run(["make", "-s", "-C", csrc, "-j8", "sanitize"], check=True)
    subprocess.run(["make", "-s", "-C", orc, "sanitize"], check=True)
    env = dict(os.environ,
               DECIDE_HIP_LIBRARY=os.path.join(csrc, "_build_san", "libdecide_hip_san.so"),
               ORACLE_LIBRARY=os.path.join(orc, "_san", "liboracle_san.so"),
               LD_PRELOAD=rt,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               DN_UNDER_SANITIZER="1")
    r = subprocess.run([sys.executable, "-m", "pytest", os.path.join(ROOT, "tests"), "-m", "not gpu", "-x", "-q",
                        "-p", "no:cacheprovider", "--deselect",
                        "tests/test_sanitizers.py::test_cpu_suite_under_asan_ubsan"],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = r.stdout + r.stderr
    print(out[-3000:])
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out
    assert r.returncode == 0
    assert " passed" in out and " failed" not in out

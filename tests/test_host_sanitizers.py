"""The C ABI's host code under AddressSanitizer and UBSan (no GPU needed).

The library is rebuilt with the sanitizers on the host pass of its C-ABI file
(``mfattn.build.build_sanitized``) and the host-side tests -- every argument
check, workspace size and plan layout the ABI computes, through ctypes and
through the torch binding's validation -- run in a child process that
preloads the sanitizer runtime and loads that build (``MFATTN_LIB``).  Any
out-of-bounds access, use after free or undefined behaviour in the host code
they reach ends the child with a report, which fails this test.
"""

import os
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def test_host_checks_are_clean_under_asan_and_ubsan():
    from mfattn import build

    runtime = build.sanitizer_runtime()
    if runtime is None:
        pytest.skip("no clang AddressSanitizer runtime under /opt/rocm/llvm")
    lib = build.build_sanitized()
    env = dict(os.environ,
               LD_PRELOAD=str(runtime),
               MFATTN_LIB=str(lib),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    which = subprocess.run(
        [sys.executable, "-c", "import mfattn._lib as L; print(L.LIB_PATH)"],
        cwd=ROOT / "minifield-training_amd", env=env, capture_output=True, text=True, timeout=300)
    assert which.returncode == 0 and which.stdout.strip() == str(lib), which.stderr[-2000:]
    proc = subprocess.run(
        [sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
         "tests/test_abi.py", "tests/test_host_checks.py"],
        cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    report = proc.stdout[-3000:] + proc.stderr[-3000:]
    assert "AddressSanitizer" not in proc.stderr and "runtime error" not in proc.stderr, report
    assert proc.returncode == 0 and "passed" in proc.stdout, report

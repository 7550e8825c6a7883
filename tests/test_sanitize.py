"""The host-side C++ under AddressSanitizer and UndefinedBehaviorSanitizer
(CPU only): a variant of libgossmx.so whose host code is instrumented
(gpt-oss-rs_amd/build.py --sanitize; the device code is the product's) and
the oracle built the same way (oracle/Makefile `san`) run the CPU suites that
drive them: the store's GOSSMX4 and SafeTensors parsers with truncated and
corrupted files, the dense path's attention, RoPE and greedy selection, the
boundary checks, and the oracle's own tests. A sanitizer report fails the
child process and this test."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "gpt-oss-rs_amd"))

import build as package_build  # noqa: E402  (gpt-oss-rs_amd/build.py)

SUITES = ["tests/test_store.py", "tests/test_dense.py", "tests/test_boundary.py", "tests/test_oracle.py"]


def _stale(target: str, sources: list[str]) -> bool:
    return not os.path.exists(target) or any(os.path.getmtime(s) > os.path.getmtime(target) for s in sources)


def test_host_code_under_address_and_ub_sanitizers():
    runtime = package_build.asan_runtime()
    if runtime is None:
        pytest.skip("the clang ASan runtime is not installed")
    csrc = os.path.join(ROOT, "gpt-oss-rs_amd", "csrc")
    srcs = [os.path.join(csrc, f) for f in os.listdir(csrc) if f.endswith((".hip", ".cpp", ".h"))]
    if _stale(package_build.SAN_LIB, srcs):
        package_build.build_sanitized()
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "san"], check=True)
    env = dict(os.environ,
               LD_PRELOAD=runtime,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               GOSSMX_LIB=package_build.SAN_LIB,
               ORACLE_LIB=os.path.join(ROOT, "oracle", "_build", "san", "libgossmx_oracle.so"))
    # The exhaustive expf comparison (2^32 calls) is left to the plain run.
    cmd = [sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
           "-k", "not every_float", *SUITES]
    res = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    report = (res.stdout + res.stderr)[-6000:]
    assert res.returncode == 0, report
    assert "ERROR: AddressSanitizer" not in report and "runtime error:" not in report, report

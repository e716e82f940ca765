"""Host sanitizer runs (CPU only): the C ABI's host code under AddressSanitizer
and UndefinedBehaviorSanitizer while a fuzzer drives every validation,
workspace query and entry point with random parameter structs
(tests/sanitize/abi_fuzz.cpp), and the CPU oracle under ASan + UBSan and
under ThreadSanitizer (tests/sanitize/oracle_run.cpp), and the kernels'
host-computed fast division against / under UBSan (tests/sanitize/fastdiv_check.cpp),
and the split plan's planner against its invariants under ASan + UBSan
(tests/sanitize/split_plan_check.cpp), the stream entries' stream-device
rule under UBSan (tests/sanitize/launch_device_check.cpp), and the main
kernel's job map -- a bijection onto (group, position), parts pinned to one
XCD, longest jobs first when interleaved -- under UBSan
(tests/sanitize/job_map_check.cpp).  Built by
tests/sanitize/Makefile."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = os.path.join(ROOT, "tests", "sanitize")
OUT = os.path.join(SAN, "_build")
REPORTS = ("ERROR: AddressSanitizer", "runtime error:", "WARNING: ThreadSanitizer",
           "ERROR: LeakSanitizer")


@pytest.fixture(scope="module")
def built():
    if shutil.which("make") is None or not os.path.exists("/opt/rocm/llvm/bin/clang++"):
        pytest.skip("no toolchain")
    r = subprocess.run(["make", "-C", SAN, "-j3"], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return OUT


@pytest.mark.parametrize("exe,args", [("abi_asan", ["20000"]), ("oracle_asan", []),
                                      ("oracle_tsan", []), ("fastdiv_ubsan", []),
                                      ("split_plan_asan", []), ("launch_device_ubsan", []),
                                      ("job_map_ubsan", [])])
def test_sanitized_run_is_clean(built, exe, args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1",
               TSAN_OPTIONS="halt_on_error=1")
    r = subprocess.run([os.path.join(built, exe), *args], capture_output=True, text=True,
                       timeout=600, env=env)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-3000:]
    for rep in REPORTS:
        assert rep not in out, out[-3000:]

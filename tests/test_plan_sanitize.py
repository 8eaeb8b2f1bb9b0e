"""The work planner (d2-sd_amd/csrc/plan.cpp) under AddressSanitizer and
UBSan on the host: tests/sanitize/fuzz_plan.cpp plans randomized batches
(ragged and empty requests, prefixes to 300K keys, page sizes 1-64 and
contiguous, two-segment prefixes, windows, every head and wave shape, split
caps, CU counts) and checks each plan's invariants; any memory error or
undefined behaviour aborts the run.  CPU only."""
import os
import shutil
import subprocess
import tempfile
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_planner_under_address_and_ub_sanitizers():
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no g++")
    with tempfile.TemporaryDirectory() as tmp:
        exe = os.path.join(tmp, "fuzz_plan")
        cmd = [cxx, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
               "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", f"-I{ROOT / 'include'}",
               f"-I{ROOT / 'd2-sd_amd' / 'csrc'}", str(ROOT / "tests" / "sanitize" / "fuzz_plan.cpp"),
               str(ROOT / "d2-sd_amd" / "csrc" / "plan.cpp"), "-o", exe]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0 and ("asan" in r.stderr.lower() or "sanitizer" in r.stderr.lower()):
            pytest.skip("sanitizer runtimes unavailable: " + r.stderr[-300:])
        assert r.returncode == 0, r.stderr[-2000:]
        env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
        r = subprocess.run([exe, "400"], capture_output=True, text=True, env=env, timeout=300)
        assert r.returncode == 0 and r.stdout.startswith("ok:"), (r.stdout[-1000:], r.stderr[-3000:])

"""The library's host-only code (JSON / manifest / tensor-file loaders, tokenizer runtime and chat template, group-64
packer, seeded generators, error reporting) and the CPU oracle, built with g++ under AddressSanitizer and
UndefinedBehaviorSanitizer (tests/sanitize/Makefile) and driven by tests/sanitize/host_checks.cpp. Any sanitizer
report aborts the program. The HIP translation units are not part of this build."""
import shutil
import subprocess
from pathlib import Path

import pytest

SAN = Path(__file__).resolve().parent / "sanitize"


def test_host_code_under_asan_ubsan(tmp_path):
    if shutil.which("g++") is None or shutil.which("make") is None:
        pytest.skip("g++ / make not available")
    b = subprocess.run(["make", "-s", "-j8", "-C", str(SAN)], capture_output=True, text=True, timeout=600)
    if b.returncode != 0 and ("asan" in b.stderr or "ubsan" in b.stderr):
        pytest.skip("sanitizer runtimes not installed: " + b.stderr[-300:])
    assert b.returncode == 0, b.stderr[-3000:]
    r = subprocess.run([str(SAN / "_build" / "host_checks"), str(tmp_path)], capture_output=True, text=True,
                       timeout=300, env={"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0",
                                         "UBSAN_OPTIONS": "print_stacktrace=1", "PATH": "/usr/bin:/bin"})
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-6000:]
    assert "host_checks: all passed" in r.stdout

"""Runs the C++ host-interface test program (tests/cpp/test_generation_context.cpp) on the GPU."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "cpp" / "test_generation_context"


def test_generation_context_cpp():
    assert EXE.exists(), "build it with `python -m soc_amd.build` (build_cpp_tests)"
    r = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "test_generation_context passed" in r.stdout

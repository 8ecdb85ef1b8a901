"""Builds soc_amd/libsoc_hip.so (HIP kernels for gfx950 + host runtime + C ABI) in-tree with hipcc.

Usage: python -m soc_amd.build [-v]

Every translation unit under soc_amd/csrc is compiled to an object in soc_amd/_build/ (in parallel) and linked into
one shared library next to this file, so that the library travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libsoc_hip.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming packed fp32 VALU instructions.
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]


def _sources() -> list[Path]:
    return sorted([p for p in CSRC.iterdir() if p.suffix in (".hip", ".cpp")])


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD / (src.stem + ".o")
    lang = ["-x", "hip"] if src.suffix in (".hip", ".cpp") else []
    cmd = [HIPCC, *COMMON, *lang, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in (r.stderr or "").splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if verbose and err.strip():
        print(err, flush=True)
    return obj


def build(verbose: bool = False) -> Path:
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    BUILD.mkdir(exist_ok=True)
    srcs = _sources()
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objs), "-lpthread"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


CPP_TESTS = ROOT / "tests" / "cpp"
APPS = PKG / "apps"


def build_cpp_tests(verbose: bool = False) -> list[Path]:
    """Host-only C++ programs that drive the C++ host interface (include/soc/gpu/runtime.h) through the library: the
    tests under tests/cpp and the programs under soc_amd/apps (soc_generate: generation through GenerationContext)."""
    outs = []
    for src in sorted(CPP_TESTS.glob("*.cpp")) + sorted(APPS.glob("*.cpp")):
        exe = src.with_suffix("") if src.parent == CPP_TESTS else src.with_name("soc_" + src.stem)
        cmd = ["g++", "-O2", "-std=c++17", f"-I{ROOT / 'include'}", str(src), f"-L{PKG}", "-lsoc_hip",
               f"-Wl,-rpath,{PKG}", "-o", str(exe)]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"g++ failed for {src.name}:\n{r.stderr}")
        outs.append(exe)
    return outs


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    print(build_cpp_tests(verbose="-v" in sys.argv))

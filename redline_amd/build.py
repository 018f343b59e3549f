"""Builds redline_amd/librlk.so (gfx950 HIP kernels + C ABI) with hipcc.

Usage: python -m redline_amd.build   (or redline_amd.build.build_library()).
The library is built in-tree so that it travels with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_obj"
LIB = PKG / "librlk.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = ["elementwise.hip", "rope_kv.hip", "attention.hip", "prefill.hip", "gemv_w4.hip", "host.cpp",
           "status.cpp"]

COMMON = [
    "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wextra",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]
# Device code: gfx950 only; packed-fp32 instructions disabled (they have
# produced sporadic wrong results on this hardware pool).
DEVICE = [
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


def _compile(src: str) -> Path:
    out = OBJ / (src + ".o")
    cmd = [HIPCC, *COMMON]
    if src.endswith(".hip"):
        cmd += [*DEVICE, "-x", "hip"]
    cmd += ["-c", str(CSRC / src), "-o", str(out)]
    subprocess.run(cmd, check=True)
    return out


def _stale(src: str) -> bool:
    """True when the object is older than its source or than any header."""
    out = OBJ / (src + ".o")
    if not out.exists():
        return True
    deps = [CSRC / src, *CSRC.glob("*.hpp"), *(ROOT / "include").rglob("*.h")]
    return max(p.stat().st_mtime for p in deps) > out.stat().st_mtime


def build_library(verbose: bool = True, only_changed: bool = False) -> Path:
    """Compiles every source (or, with only_changed, those whose object is
    stale) and links librlk.so."""
    OBJ.mkdir(exist_ok=True)
    todo = [s for s in SOURCES if not only_changed or _stale(s)]
    with ThreadPoolExecutor(max_workers=4) as pool:
        list(pool.map(_compile, todo))
    objs = [OBJ / (s + ".o") for s in SOURCES]
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", str(LIB), *map(str, objs)]
    subprocess.run(cmd, check=True)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


TEST_PROGRAMS = {"kernels_gpu": ROOT / "tests" / "cpp" / "kernels_gpu_main.cpp"}
TEST_BIN = ROOT / "tests" / "cpp" / "bin"


def build_test_programs(verbose: bool = True) -> None:
    """Compiles the C++ test programs that link librlk.so through the C++
    header (tests/cpp/*_main.cpp) into tests/cpp/bin/, with an rpath relative
    to the program so the tree can move (it runs on the GPU box)."""
    TEST_BIN.mkdir(parents=True, exist_ok=True)
    for name, src in TEST_PROGRAMS.items():
        out = TEST_BIN / name
        subprocess.run([HIPCC, "-O2", "-std=c++17", f"-I{ROOT / 'include'}", str(src), "-o", str(out),
                        f"-L{PKG}", "-lrlk", "-Wl,-rpath,$ORIGIN/../../../redline_amd"], check=True)
        if verbose:
            print(f"built {out}", file=sys.stderr)


if __name__ == "__main__":
    build_library(only_changed="--changed" in sys.argv)
    build_test_programs()

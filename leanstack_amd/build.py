"""Build libleanstack_amd.so in-tree with hipcc for gfx950.

The library is plain HIP C++ behind a C ABI (include/leanstack_amd.h); it is
loaded with ctypes after ``import torch`` so that it shares torch's HIP
runtime (both resolve the SONAME libamdhip64.so.7).

Usage: ``python -m leanstack_amd.build`` or ``build_library()``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
INCLUDE = REPO_ROOT / "include"
BUILD_DIR = PACKAGE_DIR / "_build"
LIBRARY = PACKAGE_DIR / "libleanstack_amd.so"

SOURCES = ("abi.cpp", "host_rules.cpp", "decode.hip", "skinny.hip", "gemm.hip", "stack.hip", "attention.hip",
           "noalloc.hip", "probe.hip")
OFFLOAD_ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming packed FP32 VALU ops.
HIPCC_FLAGS = (
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
)


def hipcc_path() -> str:
    found = shutil.which("hipcc")
    if found:
        return found
    candidate = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc"
    if candidate.exists():
        return str(candidate)
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{stderr}")
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr)


def build_library(verbose: bool = False, jobs: int = 4) -> Path:
    """Compile every source for gfx950 and link the shared library."""
    hipcc = hipcc_path()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    objects = [BUILD_DIR / (Path(src).name + ".o") for src in SOURCES]

    def compile_one(pair: tuple[str, Path]) -> None:
        src, obj = pair
        _run([hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(CSRC / src), "-o", str(obj)], verbose)

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        list(pool.map(compile_one, zip(SOURCES, objects)))
    tmp = LIBRARY.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)], verbose)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    path = build_library(verbose="-v" in sys.argv)
    print(path)

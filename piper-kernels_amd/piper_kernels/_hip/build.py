"""Compile ``libpiper_mi355x.so`` (gfx950) from ``piper-kernels_amd/csrc`` with hipcc.

The library is a plain C-ABI shared object (no torch headers); it is built in-tree next
to this file so it travels with the repository.  ``python -m piper_kernels._hip.build``
rebuilds it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parents[2]  # piper-kernels_amd/
CSRC = PACKAGE_ROOT / "csrc"
INCLUDE = PACKAGE_ROOT.parent / "include"
BUILD_DIR = PACKAGE_ROOT / "_build"
LIBRARY_PATH = Path(__file__).resolve().parent / "libpiper_mi355x.so"
SOURCES = ("abi.hip", "prep.hip", "attention.hip", "sage2pp.hip", "probe.hip")
OFFLOAD_ARCH = "gfx950"

COMPILE_FLAGS = (
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Packed FP32 VALU forms are kept out of generated code on this platform.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
)


def hipcc() -> str:
    candidates = [os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"]
    for candidate in candidates:
        if candidate and Path(candidate).exists():
            return candidate
    raise FileNotFoundError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd: list[str], verbose: bool) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    messages = "\n".join(
        line for line in (result.stdout + result.stderr).splitlines() if noise not in line
    ).strip()
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(cmd)}\n{messages}")
    if verbose and messages:
        print(messages, file=sys.stderr)


def build_library(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link the shared library; returns its path."""
    compiler = hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    includes = [f"-I{INCLUDE}", f"-I{CSRC}"]
    objects = [BUILD_DIR / (Path(s).stem + ".o") for s in SOURCES]

    def compile_one(pair: tuple[str, Path]) -> None:
        source, obj = pair
        _run([compiler, *COMPILE_FLAGS, *includes, "-c", str(CSRC / source), "-o", str(obj)], verbose)

    with ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        list(pool.map(compile_one, zip(SOURCES, objects)))
    tmp = LIBRARY_PATH.with_suffix(f".so.tmp{os.getpid()}")
    _run([compiler, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)], verbose)
    os.replace(tmp, LIBRARY_PATH)
    return LIBRARY_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))

"""Compile the gfx950 libraries from ``piper-kernels_amd/csrc`` with hipcc.

``libpiper_mi355x.so`` is the operator's C ABI (``include/piper_mi355x.h``); ``libpiper_probe.so``
holds the measurement probes (``include/piper_probe.h``), which only bench.py and the tests load.
Both are plain C-ABI shared objects (no torch headers), built in-tree next to this file so they
travel with the repository.  ``python -m piper_kernels._hip.build`` rebuilds them.
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
PROBE_LIBRARY_PATH = Path(__file__).resolve().parent / "libpiper_probe.so"
SOURCES = ("abi.hip", "prep.hip", "attention.hip", "sage2pp.hip")
PROBE_SOURCES = ("probe.hip",)
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


def _link(compiler: str, objects: list[Path], target: Path, verbose: bool) -> None:
    tmp = target.with_suffix(f".so.tmp{os.getpid()}")
    _run([compiler, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)], verbose)
    os.replace(tmp, target)


def build_library(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link both libraries; returns the operator
    library's path (the probe library is ``PROBE_LIBRARY_PATH``)."""
    compiler = hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    includes = [f"-I{INCLUDE}", f"-I{CSRC}"]
    sources = SOURCES + PROBE_SOURCES
    objects = {s: BUILD_DIR / (Path(s).stem + ".o") for s in sources}

    def compile_one(source: str) -> None:
        _run([compiler, *COMPILE_FLAGS, *includes, "-c", str(CSRC / source), "-o", str(objects[source])], verbose)

    with ThreadPoolExecutor(max_workers=len(sources)) as pool:
        list(pool.map(compile_one, sources))
    _link(compiler, [objects[s] for s in SOURCES], LIBRARY_PATH, verbose)
    _link(compiler, [objects[s] for s in PROBE_SOURCES], PROBE_LIBRARY_PATH, verbose)
    return LIBRARY_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))

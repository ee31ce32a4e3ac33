"""bench.py's command-line contract, without a GPU: the one-GPU refusal and the workload list."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _run(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_is_refused_with_a_message() -> None:
    result = _run("--gpus", "2")
    assert result.returncode == 2
    assert "exactly one GPU" in result.stderr and result.stdout == ""


def test_workloads_are_the_baseline_configs_and_the_reference_shape() -> None:
    result = _run("--help")
    assert result.returncode == 0
    for name in ("c1", "c2", "c3", "c4", "c5", "r1", "r2"):
        assert name in result.stdout


def test_reference_figures_match_the_baseline_document() -> None:
    """The r1 comparison divides by the reference's published complete-call rate."""
    sys.path.insert(0, str(ROOT))
    import bench

    from piper_kernels.workloads import WORKLOADS

    for name, ref in bench.REFERENCE_PUBLISHED.items():
        b, h, sq, sk, d = WORKLOADS[name].shape
        ops = 4 * b * h * sq * sk * d
        assert abs(ops / (ref["complete_ms"] * 1e-3) / 1e12 - ref["complete_tops"]) < 0.5, name
        assert abs(ops / (ref["hot_ms"] * 1e-3) / 1e12 - ref["hot_tops"]) < 0.5, name
    assert WORKLOADS["r2"].shape == (1, 1, 131072, 131072, 128) and not WORKLOADS["r2"].is_causal


def test_source_digest_identifies_the_tree() -> None:
    """The record's code identity without git: stable across calls, hex SHA-256 values."""
    sys.path.insert(0, str(ROOT))
    import bench

    first, second = bench.source_digest(), bench.source_digest()
    assert first == second
    assert len(first["sources_sha256"]) == 64 and int(first["sources_sha256"], 16) >= 0
    assert first["library_sha256"] is None or len(first["library_sha256"]) == 64

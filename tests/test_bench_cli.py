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
    for name in ("c1", "c2", "c3", "c4", "c5", "r1"):
        assert name in result.stdout


def test_reference_figures_match_the_baseline_document() -> None:
    """The r1 comparison divides by the reference's published complete-call rate."""
    sys.path.insert(0, str(ROOT))
    import bench

    ref = bench.REFERENCE_R1
    ops = 4 * 1 * 8 * 8192 * 8192 * 128
    assert abs(ops / (ref["complete_ms"] * 1e-3) / 1e12 - ref["complete_tops"]) < 0.5
    assert abs(ops / (ref["hot_ms"] * 1e-3) / 1e12 - ref["hot_tops"]) < 0.5


def test_source_digest_identifies_the_tree() -> None:
    """The record's code identity without git: stable across calls, hex SHA-256 values."""
    sys.path.insert(0, str(ROOT))
    import bench

    first, second = bench.source_digest(), bench.source_digest()
    assert first == second
    assert len(first["sources_sha256"]) == 64 and int(first["sources_sha256"], 16) >= 0
    assert first["library_sha256"] is None or len(first["library_sha256"]) == 64

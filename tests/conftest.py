"""Shared pytest setup: import paths, the ``gpu`` marker and device helpers."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
for entry in (REPO, REPO / "piper-kernels_amd"):
    if str(entry) not in sys.path:
        sys.path.insert(0, str(entry))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an AMD gfx950 (MI355X) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gfx950_device():
    """The MI355X device for GPU tests; fails (not skips) when the HIP library is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from piper_kernels._hip.library import load_library
    from piper_kernels._hip.targets import AcceleratorTarget

    device = torch.device("cuda", 0)
    target = AcceleratorTarget.from_device(device)
    assert target.supports_piper_mi355x, f"GPU tests need gfx950, got {target}"
    load_library()  # raises if the library is not built: GPU tests never fall back
    return device

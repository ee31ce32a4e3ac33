"""Accelerator facts needed to pick the MI355X backend.

Restates the behaviour of the reference's ``AcceleratorTarget``
(``src/piper_kernels/_triton/targets.py:8-104``): a frozen (backend, architecture)
pair, resolved from a torch device, with HIP architectures read from
``gcnArchName`` and normalised by dropping ``:feature`` suffixes.  The NVIDIA
capability helpers of the reference are not needed here; the one predicate this
backend adds is :attr:`AcceleratorTarget.supports_piper_mi355x`.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

MI355X_ARCHITECTURE = "gfx950"


def _normalize_architecture(architecture: object | None) -> str | None:
    """Lower-case, strip and drop optional ``:feature`` suffixes (targets.py:8-13)."""
    if architecture is None:
        return None
    normalized = str(architecture).strip().lower().partition(":")[0]
    return normalized or None


@dataclass(frozen=True)
class AcceleratorTarget:
    """Compiler-backend name (``cuda``/``hip``/``cpu``...) and canonical architecture."""

    backend: str
    architecture: str | None = None

    def __post_init__(self) -> None:
        object.__setattr__(self, "backend", self.backend.strip().lower())
        object.__setattr__(self, "architecture", _normalize_architecture(self.architecture))

    @classmethod
    def from_device(cls, device: torch.device) -> "AcceleratorTarget":
        """Resolve ``device`` (targets.py:31-43): HIP devices report ``gcnArchName``."""
        if device.type != "cuda":
            return cls(backend=device.type)
        if getattr(torch.version, "hip", None) is not None:
            properties = torch.cuda.get_device_properties(device)
            return cls(backend="hip", architecture=getattr(properties, "gcnArchName", None))
        major, minor = torch.cuda.get_device_capability(device)
        return cls(backend="cuda", architecture=f"sm{major}{minor}")

    @property
    def is_amd_hip(self) -> bool:
        return self.backend == "hip"

    def is_architecture(self, *architectures: str) -> bool:
        return self.architecture is not None and self.architecture in (
            _normalize_architecture(a) for a in architectures
        )

    @property
    def supports_piper_mi355x(self) -> bool:
        """Whether the hand-written gfx950 (CDNA4, MI355X) kernels can run on this target."""
        return self.is_amd_hip and self.is_architecture(MI355X_ARCHITECTURE)

"""Public entry point and backend selection for Piper Attention on MI355X.

Same signature, defaults and validation as the reference's ``piper_attention``
(``src/piper_kernels/attention/piper_attention/dispatch.py:39-83``).  The reference routes
supported NVIDIA targets to its Triton custom op and everything else to its portable
PyTorch reference.  This package *is* the gfx950 backend: a gfx950 HIP device goes to
the ``piper_kernels::piper_attention`` custom op backed by the hand-written HIP kernels;
any other device raises ``NotImplementedError`` (the portable reference stays with the
reference package, whose dispatch would route gfx950 devices to this backend), and
a gfx950 device without the built library raises instead of silently computing on the CPU.
"""

from __future__ import annotations

import torch

from ..._hip.library import load_library
from ..._hip.targets import AcceleratorTarget
from .._validation import validate_attention_inputs
from .hip import hip_piper_attention


def _validate_inputs(
    query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scale: float | None, is_causal: bool
) -> float:
    return validate_attention_inputs("Piper Attention", query, key, value, scale, is_causal)


def _supports_hip(target: AcceleratorTarget) -> bool:
    return target.supports_piper_mi355x


def piper_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    scale: float | None = None,
    is_causal: bool = False,
) -> torch.Tensor:
    """Run Piper Attention's key-scaled UINT8-P/INT8-V forward attention on MI355X.

    Query, key, and value use ``[batch, heads, sequence, head_dim]`` layout with FP16 or
    BF16 elements and contiguous head dimensions (64 or 128). Query and key sequence
    lengths may differ for non-causal attention. ``scale`` defaults to ``head_dim**-0.5``.

    K is smoothed by its sequence mean and Q/K are quantised to INT8 with one scale per
    thread group of each 32-row (Q) or 64-row (K) block, the granularity of the reference's
    portable path; each V row gets its own signed-INT8 scale, folded into UINT8 probability
    codes.
    Non-causal calls centre V by its sequence-wide per-feature mean and restore it in the
    epilogue; causal calls stay uncentred. Inference only.
    """
    converted_scale = _validate_inputs(query, key, value, scale, is_causal)
    target = AcceleratorTarget.from_device(query.device)
    if not _supports_hip(target):
        raise NotImplementedError(
            "this Piper Attention build runs only on AMD gfx950 (MI355X) HIP devices; "
            f"got backend={target.backend!r} architecture={target.architecture!r}"
        )
    if not torch.compiler.is_compiling():
        load_library()  # raises LibraryUnavailableError (a RuntimeError) if the library is missing
    return hip_piper_attention(query, key, value, converted_scale, is_causal)

"""Public entry point and backend selection for SageAttention2++ on MI355X.

Same signature, defaults and validation as the reference's ``sage_attention_2pp``
(``src/piper_kernels/attention/sage_attention_2pp/dispatch.py:39-64``).  The reference routes
NVIDIA targets with FP8 tensor cores to its Triton custom op and everything else to its
portable PyTorch reference.  This package is the gfx950 backend: a gfx950 HIP device goes to
the ``piper_kernels::sage_attention_2pp`` custom op backed by the HIP kernels (FP8 E4M3 PV on
``v_mfma_f32_32x32x64_f8f6f4``); any other device raises ``NotImplementedError``, and a gfx950
device without the built library raises instead of computing on the CPU.
"""

from __future__ import annotations

import torch

from ..._hip.library import load_library
from ..._hip.targets import AcceleratorTarget
from .._validation import validate_attention_inputs
from .hip import hip_sage_attention_2pp


def _validate_inputs(
    query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scale: float | None, is_causal: bool
) -> float:
    return validate_attention_inputs("SageAttention2++", query, key, value, scale, is_causal)


def _supports_hip(target: AcceleratorTarget) -> bool:
    return target.supports_piper_mi355x


def sage_attention_2pp(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    scale: float | None = None,
    is_causal: bool = False,
) -> torch.Tensor:
    """Run canonical SageAttention2++ 8+8 forward attention on MI355X.

    Query, key, and value use ``[batch, heads, sequence, head_dim]`` layout with FP16 or BF16
    elements and contiguous head dimensions (64 or 128). Query and key sequence lengths may
    differ for non-causal attention. ``scale`` defaults to ``head_dim**-0.5``.

    Q/K are INT8 (K smoothed by its sequence mean; one scale per 32 query rows and per 64 key
    rows), V is FP8 E4M3 with one scale per channel, probabilities are FP8 E4M3 in a softmax
    frame shifted by ln 448. The PV products accumulate in FP32 (gfx950's FP8 MFMA), where the
    reference rounds each 64-key partial to FP16. Inference only.
    """
    converted_scale = _validate_inputs(query, key, value, scale, is_causal)
    target = AcceleratorTarget.from_device(query.device)
    if not _supports_hip(target):
        raise NotImplementedError(
            "this SageAttention2++ build runs only on AMD gfx950 (MI355X) HIP devices; "
            f"got backend={target.backend!r} architecture={target.architecture!r}"
        )
    if not torch.compiler.is_compiling():
        load_library()  # raises LibraryUnavailableError (a RuntimeError) if the library is missing
    return hip_sage_attention_2pp(query, key, value, converted_scale, is_causal)

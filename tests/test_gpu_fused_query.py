"""The fused entry point (query quantised in the attention prologue) against the two-step path.

``piper_attention_forward_fused`` must quantise each 32-row query block with the prep's own
arithmetic, so its output equals ``piper_prepare`` + ``piper_attention_forward`` bit for bit
(FP32 and 16-bit outputs) on every shape class the reference tests: ragged lengths, causal
masks, both input dtypes, D = 64 and 128, every launch plan, strided query views and blocks
that quantise to all-zero or saturated codes.  A prep that skips the query must still write
the same K/V operands.
"""

from __future__ import annotations

import pytest
import torch

from _parity import gpu_attention, gpu_prepare, log
from piper_kernels.attention.piper_attention._plan import MI355XPlan

pytestmark = pytest.mark.gpu

SHAPES = [
    # (B, H, Sq, Sk, D, dtype, causal)
    (1, 2, 256, 256, 128, torch.float16, False),
    (2, 3, 35, 67, 64, torch.bfloat16, False),
    (1, 2, 300, 300, 128, torch.float16, True),
    (1, 3, 700, 700, 64, torch.bfloat16, True),
    (1, 1, 1, 1, 64, torch.float16, False),
    (2, 2, 1000, 333, 128, torch.bfloat16, False),
]


def _inputs(shape, seed):
    b, h, sq, sk, d, dtype, _ = shape
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, h, sq, d, generator=g).to(dtype)
    k = (torch.randn(b, h, sk, d, generator=g) + 0.5 * torch.randn(b, h, 1, d, generator=g)).to(dtype)
    v = (torch.randn(b, h, sk, d, generator=g) + 2.0 * torch.randn(b, h, 1, d, generator=g)).to(dtype)
    return q, k, v


def _both(q, k, v, causal, device, plan=None):
    d = q.shape[-1]
    two_step = gpu_prepare(q, k, v, d**-0.5, causal, device, plan=plan)
    fused = gpu_prepare(q, k, v, d**-0.5, causal, device, plan=plan, quantize_query=False)
    assert fused.fused_query and fused.query_code is None and not two_step.fused_query
    return two_step, fused


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(str(x) for x in s[:5]) + f"-{str(s[5])[6:]}-c{int(s[6])}")
def test_fused_query_matches_two_step_bitwise(gfx950_device, shape) -> None:
    log(f"[fused] shape {shape}")
    q, k, v = _inputs(shape, seed=71)
    two_step, fused = _both(q, k, v, shape[6], gfx950_device)
    for dtype in (torch.float32, shape[5]):
        expected = gpu_attention(two_step, dtype)
        actual = gpu_attention(fused, dtype)
        assert torch.equal(actual, expected), f"{dtype}: max diff {(actual.float() - expected.float()).abs().max()}"
    # the K/V operands do not depend on the query flag
    assert torch.equal(fused.key_code(), two_step.key_code())
    assert torch.equal(fused.key_scale, two_step.key_scale)
    assert torch.equal(fused.value_code_transposed(), two_step.value_code_transposed())
    assert torch.equal(fused.value_log2_scale(), two_step.value_log2_scale())
    assert torch.equal(fused.value_correction(), two_step.value_correction())
    assert torch.equal(fused.value_mean, two_step.value_mean)


def test_fused_query_every_plan(gfx950_device) -> None:
    q, k, v = _inputs((1, 2, 700, 700, 128, torch.float16, True), seed=72)
    reference = None
    for plan in MI355XPlan.all_plans():
        log(f"[fused] plan {plan.plan_id}")
        two_step, fused = _both(q, k, v, True, gfx950_device, plan=plan)
        out = gpu_attention(fused)
        assert torch.equal(out, gpu_attention(two_step))
        if reference is None:
            reference = out
        assert torch.equal(out, reference)


def test_fused_query_extreme_blocks(gfx950_device) -> None:
    """An all-zero query block (scale 1e-7, codes 0), a block holding the fp16 maximum and a
    block of sub-normal values quantise exactly as in the prep."""
    q, k, v = _inputs((1, 1, 128, 128, 128, torch.float16, False), seed=73)
    q[:, :, 0:32] = 0
    q[:, :, 32:64, 5] = 65504.0
    q[:, :, 64:96] = q[:, :, 64:96] * 2.0**-20
    two_step, fused = _both(q, k, v, False, gfx950_device)
    assert torch.equal(gpu_attention(fused), gpu_attention(two_step))


def test_fused_query_strided_view(gfx950_device) -> None:
    """A [B, S, H, D] projection read through a transposed view, with no copy."""
    torch.manual_seed(74)
    base = torch.randn(2, 200, 3, 4, 128, dtype=torch.bfloat16, device=gfx950_device)
    q, k, v = (base[:, :, i].transpose(1, 2) for i in range(3))
    two_step, fused = _both(q, k, v, False, gfx950_device)
    assert fused.query.data_ptr() == q.data_ptr()
    assert torch.equal(gpu_attention(fused), gpu_attention(two_step))

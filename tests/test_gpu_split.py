"""The key-range split plans on MI355X: parity with the oracle and with the unsplit kernel.

A split plan cuts each query tile's key tiles into ranges, one workgroup each; every workgroup
runs the reference recurrence (reference.py:61-118) over its range and writes its unnormalised
numerator, denominator and reference maximum, and a merge kernel aligns the parts' maxima and
adds them.  The parts' sums are combined in another order than one sequential pass, so the
outputs equal the unsplit plans' only to rounding: they are held to the oracle's parity gate,
and to a tight distance from the unsplit kernel.  Ragged key ranges, a single key tile (the
split degenerates to one part), both Q/K granularities, both head sizes, the fused and two-step
entry points and every output dtype are covered, and so is the reference's long-sequence
shape B1 H1 N131072 D128 (benchmarks/README.md:526) on row slices.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _parity import assert_attention_close, gpu_attention, gpu_prepare, log, oracle_attention
from oracle import piper_oracle as oracle
from piper_kernels.attention.piper_attention._plan import MI355XPlan
from piper_kernels.workloads import WORKLOADS, make_inputs

pytestmark = pytest.mark.gpu

UNSPLIT = MI355XPlan(waves=4, three_per_cu=True)

CASES = [
    # (B, H, Sq, Sk, D, dtype, parts, granularity)
    (1, 2, 1000, 1000, 128, torch.float16, 3, "per_thread"),  # 16 key tiles: 6 + 6 + 4
    (2, 1, 300, 4100, 64, torch.bfloat16, 8, "per_thread"),  # 65 tiles: 7 x 9 + 2
    (1, 3, 257, 640, 128, torch.bfloat16, 5, "per_warp"),  # 10 tiles: 5 x 2
    (1, 1, 64, 64, 128, torch.float16, 4, "per_thread"),  # one tile: a single part
    (1, 2, 128, 4096, 128, torch.float16, 2, "per_warp"),
]


def _inputs(case, seed):
    b, h, sq, sk, d, dtype, _, _ = case
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((b, h, sq, d), generator=g).to(dtype)
    k = (torch.randn((b, h, sk, d), generator=g) + torch.randn((b, h, 1, d), generator=g)).to(dtype)
    v = (torch.randn((b, h, sk, d), generator=g) + 2 * torch.randn((b, h, 1, d), generator=g)).to(dtype)
    return q, k, v


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}x{c[3]}x{c[4]}-p{c[6]}-{c[7]}")
def test_split_plans_meet_the_oracle_and_track_the_unsplit_kernel(case, gfx950_device) -> None:
    b, h, sq, sk, d, dtype, parts, granularity = case
    scale = d**-0.5
    plan = MI355XPlan(waves=4, three_per_cu=True, key_parts=parts)
    log(f"[case] key-range split {case}")
    q, k, v = _inputs(case, 900 + parts)
    fused = gpu_prepare(q, k, v, scale, False, gfx950_device, plan=plan, quantize_query=False,
                        qk_granularity=granularity)
    out32 = gpu_attention(fused, torch.float32)
    # the two-step entry point (prepared query codes) runs the same split bit for bit
    two_step = gpu_prepare(q, k, v, scale, False, gfx950_device, plan=plan, qk_granularity=granularity)
    assert torch.equal(gpu_attention(two_step, torch.float32), out32)
    # 16-bit outputs are the RNE rounding of the merged FP32 result
    out16 = gpu_attention(fused, dtype)
    assert torch.equal(out16, out32.to(dtype))
    got = out32.cpu().numpy()
    expected, bound = oracle_attention(oracle.prepare(q, k, v, False, granularity), scale, False)
    assert_attention_close(got, expected, f"split {parts} parts", flip_bound=bound)
    unsplit = gpu_prepare(q, k, v, scale, False, gfx950_device, plan=UNSPLIT, quantize_query=False,
                          qk_granularity=granularity)
    reference = gpu_attention(unsplit, torch.float32).cpu().numpy()
    diff = np.abs(got - reference).max()
    log(f"  max |split - unsplit| = {diff:.3e}")
    assert diff <= 1e-5 * max(1.0, float(np.abs(reference).max()))
    if -(-sk // 64) == 1:  # one key tile: nothing to split, the unsplit kernel runs
        assert np.array_equal(got, reference)


def test_split_preserves_constant_value_rows_exactly(gfx950_device) -> None:
    """A constant V is centred to zero codes: every part's numerator is zero, and the merged
    output is the mean, exactly (reference.py:42-57's property, across the merge)."""
    torch.manual_seed(5)
    q = torch.randn(1, 2, 300, 128).to(torch.float16)
    k = torch.randn(1, 2, 2000, 128).to(torch.float16)
    v = torch.randn(1, 2, 1, 128).expand(1, 2, 2000, 128).contiguous().to(torch.float16)
    plan = MI355XPlan(waves=4, three_per_cu=True, key_parts=6)
    log("[case] split, constant V")
    out = gpu_attention(gpu_prepare(q, k, v, 128**-0.5, False, gfx950_device, plan=plan, quantize_query=False),
                        torch.float32).cpu()
    assert torch.equal(out, v[:, :, :1].float().expand_as(out))


@pytest.mark.parametrize("plan", [MI355XPlan(waves=4, three_per_cu=True, key_parts=3), UNSPLIT],
                         ids=["split3", "unsplit"])
def test_reference_long_sequence_shape_row_slices(plan, gfx950_device) -> None:
    """B1 H1 N131072 D128 (the reference's published long-sequence point): the whole call on the
    GPU, row slices against the oracle at the operator's granularity."""
    w = WORKLOADS["r2"]
    q, k, v = make_inputs(w)
    scale = w.head_dim**-0.5
    log(f"[case] r2 {w.shape} plan={plan.plan_id}")
    prepared = gpu_prepare(q, k, v, scale, False, gfx950_device, plan=plan, quantize_query=False,
                           qk_granularity="per_thread")
    out32 = gpu_attention(prepared, torch.float32).cpu().numpy()
    assert np.isfinite(out32).all()
    prep = oracle.prepare(q, k, v, False, "per_thread")
    for rows in (slice(0, 64), slice(65536, 65600), slice(131008, 131072)):
        sub = dict(prep)
        sub["query_code"] = prep["query_code"][:, :, rows]
        sub["query_scale"] = prep["query_scale"][:, :, rows]
        expected, bound = oracle_attention(sub, scale, False, query_offset=rows.start)
        assert_attention_close(out32[:, :, rows], expected, f"r2 rows {rows.start}:{rows.stop}", flip_bound=bound)

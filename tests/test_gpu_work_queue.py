"""The work-queue plan on MI355X: bit-identical to hardware dispatch on the shapes where its queue
arithmetic has edge cases.

The plan (csrc/attention.hip, attention_w3_queue_kernel) runs a persistent grid of three
workgroups per CU that take query tiles from one queue per XCC: queue q holds a consecutive range
of the XCD-aware order's logical tile ids, each workgroup takes its first tile statically and then
claims tiles with atomics, stealing from the other queues once its own is empty.  Every tile is
computed by the same code as in the one-workgroup-per-tile kernel, so the output must equal plan
16's bit for bit whatever the claim order: fewer tiles than queues or than workgroups, tile counts
that do not divide over the queues, batch-heads not divisible by the queues (the interleaved causal
order then walks head by head), both head sizes, every output dtype, both granularities.  The
counters live in a caller workspace that the library sets before each call, so one workspace is
reused across calls of different shapes here through the C ABI.
"""

from __future__ import annotations

import pytest
import torch

from _parity import gpu_attention, gpu_prepare, log
from piper_kernels._hip import library as native
from piper_kernels.attention.piper_attention._plan import MI355XPlan

pytestmark = pytest.mark.gpu

HARDWARE = MI355XPlan(waves=4, three_per_cu=True)
QUEUE = MI355XPlan(waves=4, three_per_cu=True, work_queue=True)
QUEUE_INTERLEAVED = MI355XPlan(waves=4, three_per_cu=True, work_queue=True, causal_interleave=True)

CASES = [
    # (B, H, S, D, dtype, causal, granularity)
    (1, 1, 64, 64, torch.float16, False, "per_thread"),  # one tile: fewer tiles than queues
    (1, 1, 64, 64, torch.float16, True, "per_warp"),
    (3, 5, 1000, 128, torch.bfloat16, True, "per_thread"),  # 15 batch-heads: not divisible by 8
    (2, 8, 777, 128, torch.float16, True, "per_thread"),  # 16 batch-heads: interleaved per queue
    (2, 3, 4100, 64, torch.bfloat16, False, "per_warp"),  # 33 tiles per head
    (1, 24, 2048, 128, torch.float16, False, "per_thread"),  # 384 tiles: fewer than the 768 workers
    (4, 8, 4096, 128, torch.bfloat16, True, "per_thread"),  # 1024 tiles: more than the workers
]


def _inputs(case, seed):
    b, h, s, d, dtype, _, _ = case
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((b, h, s, d), generator=g).to(dtype)
    k = (torch.randn((b, h, s, d), generator=g) + torch.randn((b, h, 1, d), generator=g)).to(dtype)
    v = (torch.randn((b, h, s, d), generator=g) + 2 * torch.randn((b, h, 1, d), generator=g)).to(dtype)
    return q, k, v


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}x{c[3]}-{'causal' if c[5] else 'full'}-{c[6]}")
def test_work_queue_is_bit_identical_to_hardware_dispatch(case, gfx950_device) -> None:
    b, h, s, d, dtype, causal, granularity = case
    log(f"[case] work queue {case}")
    q, k, v = _inputs(case, 1200 + s + h)
    outs = {}
    for plan in (HARDWARE, QUEUE, QUEUE_INTERLEAVED):
        prepared = gpu_prepare(q, k, v, d**-0.5, causal, gfx950_device, plan=plan, quantize_query=False,
                               qk_granularity=granularity)
        outs[plan.plan_id] = [gpu_attention(prepared, out_dtype).cpu() for out_dtype in (torch.float32, dtype)]
    reference = outs[HARDWARE.plan_id]
    for plan_id, (out32, out16) in outs.items():
        assert torch.equal(out32, reference[0]), f"plan {plan_id}: FP32 output differs"
        assert torch.equal(out16, reference[1]), f"plan {plan_id}: 16-bit output differs"
    assert torch.equal(reference[1], reference[0].to(dtype))  # 16-bit = RNE of the FP32 result


def test_one_workspace_reused_across_calls_of_different_shapes(gfx950_device) -> None:
    """The library sets the queue counters on the stream before every call: a workspace left by a
    call over one shape serves the next, smaller call (and then the first shape again)."""
    from piper_kernels.attention.piper_attention.hip import _native_input

    lib = native.load_library()
    workspace = torch.empty(lib.attention_workspace_bytes(native.PiperShape(1, 1, 64, 64, 128), QUEUE.plan_id),
                            dtype=torch.uint8, device=gfx950_device)
    assert workspace.numel() == 256
    stream = torch.cuda.current_stream(gfx950_device)
    for i, case in enumerate([(2, 4, 3000, 128, torch.float16, True, "per_thread"),
                              (1, 2, 300, 128, torch.float16, False, "per_thread"),
                              (2, 4, 3000, 128, torch.float16, True, "per_thread")]):
        b, h, s, d, dtype, causal, _ = case
        log(f"[case] shared workspace call {i + 1}: {case}")
        q, k, v = _inputs(case, 1300 + i)
        prepared = gpu_prepare(q, k, v, d**-0.5, causal, gfx950_device, plan=HARDWARE, quantize_query=False,
                               qk_granularity="per_thread")
        expected = gpu_attention(prepared, torch.float32)
        out = torch.empty_like(expected)
        query, query_arg = _native_input(prepared.query)
        args = native.PiperAttentionFusedArgs(
            abi_version=native.ABI_VERSION, dtype=native.FLOAT16, output_dtype=native.FLOAT32,
            is_causal=int(causal), plan=QUEUE.plan_id, scale=d**-0.5, flags=native.ATTENTION_QK_PER_THREAD,
            reserved=0, shape=native.PiperShape(b, h, s, s, d), query=query_arg,
            prepared=prepared.native_prepared(), output=out.data_ptr(),
            workspace=workspace.data_ptr(), workspace_bytes=workspace.numel(),
        )
        lib.attention_forward_fused(args, stream.cuda_stream)
        torch.cuda.synchronize(gfx950_device)
        assert torch.equal(out, expected), f"call {i + 1} differs from hardware dispatch"

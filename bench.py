#!/usr/bin/env python3
"""Benchmark: Piper Attention forward on one MI355X (gfx950).

Workload (the headline shape): B1 H24 S16384 D128 fp16,
non-causal, synthetic seeded inputs already resident in HBM.  One *step* is one complete
operator call, exactly what ``piper_attention`` runs: the HIP prep pipeline (K/V means,
INT8 K and V quantisation) followed by the fused INT8-MFMA attention kernel, which
quantises each query block in its prologue (``--two-step``: the prep quantises Q as well
and the kernel reads the prepared query codes; the output is bit-identical).

Prints ONE JSON line.  ``value`` = whole-call TOPS (reference op count 4*B*H*Sq*Skv*D per
call, benchmarks/benchmark_attention.py:184-193).  ``roofline`` prices the dominant
kernel (the fused attention kernel) against MI355X's dense INT8 MFMA peak, with its
average duration measured by HIP events recorded on the launch stream inside the timed
region.  ``mfma_peak_measured`` is the sustained dense INT8 and FP8 MFMA rate of the same GPU
(the library's back-to-back MFMA probe, results checked), and ``attention_kernel`` also
reports the kernel's fraction of that measured INT8 rate.  ``mfma_valu_sharing`` times the same
probe's MFMA-only, FP32-FMA-only and interleaved kinds at the kernel's occupancy (two waves per
SIMD): how much MFMA execution and VALU issue overlap on this GPU.  ``cpu_baseline`` times the CPU
oracle (a numpy restatement of the reference's portable path) on a bounded slice of the same
workload, on one host thread.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c3] [--no-cpu-baseline] [--two-step]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path[:0] = [str(REPO), str(REPO / "piper-kernels_amd")]

INT8_PEAK_TOPS = 5033.2  # MI355X dense INT8 MFMA: 256 CU x 2.4 GHz x 8192 ops/clk/CU
HBM_PEAK_GBPS = 8000.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args() -> argparse.Namespace:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--workload", default="c3", choices=["c1", "c2", "c3", "c4", "c5"])
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--cpu-seconds", type=float, default=15.0, help="target CPU-baseline sample time")
    parser.add_argument(
        "--two-step", action="store_true", help="time the prep of Q, K, V + attention on prepared query codes"
    )
    parser.add_argument(
        "--qk-granularity",
        choices=["per_thread", "per_warp"],
        default="per_thread",
        help="Q/K scale granularity (the operator's default: per_thread, as the reference's portable path)",
    )
    parser.add_argument(
        "--operator",
        choices=["piper_attention", "sage_attention_2pp"],
        default="piper_attention",
        help="the operator whose complete call is a step (default: Piper Attention, the headline)",
    )
    return parser.parse_args()


def traffic_from_profile(workload: str):
    """HBM bytes per attention launch measured by rocprofv3 --pmc (committed summary), if any."""
    path = REPO / "profiles" / f"attention_{workload}_hbm_traffic.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text())["bytes_per_launch"]
    except (KeyError, ValueError):
        return None


def cpu_baseline(workload, seconds: float) -> dict:
    """Time the CPU oracle on whole (batch 0) heads of the workload until ~`seconds` elapse.

    Each head is the full reference computation for that head: prep (means, Q/K/V codes) and
    the 64-key streaming loop over every query row, numpy on one thread.
    """
    import platform

    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import piper_oracle as oracle
    from piper_kernels.measure import attention_operations
    from piper_kernels.workloads import make_inputs

    scale = workload.head_dim**-0.5
    heads = 0
    elapsed = 0.0
    with threadpool_limits(limits=1):
        while heads < workload.heads and (heads == 0 or elapsed < seconds):
            q, k, v = make_inputs(workload, heads=[heads], batches=[0])
            start = time.perf_counter()
            oracle.piper_attention_reference(q, k, v, scale, workload.is_causal, "per_thread")
            elapsed += time.perf_counter() - start
            heads += 1
            log(f"[bench] cpu baseline: {heads} head(s), {elapsed:.1f} s")
    ops = attention_operations(1, heads, workload.query_length, workload.key_length, workload.head_dim,
                               workload.is_causal)
    return {
        "value": ops / elapsed / 1e12,
        "unit": "TOPS",
        "cores": 1,
        "kind": "port",
        "sample": (
            f"{workload.name}: {heads} of {workload.batch * workload.heads} (batch, head) slices, each the full "
            f"reference computation (K/V means, per_thread Q/K codes, V codes, 64-key streaming loop over all "
            f"{workload.query_length} query rows); {elapsed:.1f} s wall; numpy {np.__version__} on 1 thread; "
            f"cpu={platform.processor() or platform.machine()} os.cpu_count={os.cpu_count()}"
        ),
    }


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py runs on exactly one GPU (asked for --gpus {args.gpus}); this build has no "
            "multi-GPU path (heads are independent: the operator would shard over (batch, head) pairs).",
            file=sys.stderr,
        )
        return 2

    import torch

    from piper_kernels.attention.piper_attention.hip import _launch_piper_attention, _prepare_piper_attention
    from piper_kernels.measure import attention_operations, prep_algorithmic_bytes, sage_prep_algorithmic_bytes
    from piper_kernels.workloads import WORKLOADS, make_inputs

    workload = WORKLOADS[args.workload]
    device = torch.device("cuda", 0)
    log(f"[bench] generating {workload.description}")
    q, k, v = make_inputs(workload, device)
    scale = workload.head_dim**-0.5
    b, h, sq, sk, d = workload.shape
    ops = attention_operations(b, h, sq, sk, d, workload.is_causal)

    sage = args.operator == "sage_attention_2pp"
    if sage:
        from piper_kernels.attention.sage_attention_2pp.hip import _launch_sage_attention_2pp as launch
        from piper_kernels.attention.sage_attention_2pp.hip import _prepare_sage_attention_2pp

        def prepare():
            return _prepare_sage_attention_2pp(q, k, v, scale, workload.is_causal)

    else:
        launch = _launch_piper_attention

        def prepare():
            return _prepare_piper_attention(
                q, k, v, scale, workload.is_causal, quantize_query=args.two_step, qk_granularity=args.qk_granularity
            )

    def step(events=None):
        if events is not None:
            events[0].record()
        prepared = prepare()
        if events is not None:
            events[1].record()
        out = launch(prepared)
        if events is not None:
            events[2].record()
        return out

    with torch.no_grad():
        log(f"[bench] warmup {args.warmup}")
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
        log(f"[bench] timing {args.steps} steps")
        torch.cuda.synchronize()
        start = time.perf_counter()
        for i in range(args.steps):
            step(events[i])
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - start

    ms_per_step = elapsed * 1e3 / args.steps
    prep_ms = sorted(e[0].elapsed_time(e[1]) for e in events)
    attn_ms = sorted(e[1].elapsed_time(e[2]) for e in events)
    attn_mean = sum(attn_ms) / len(attn_ms)
    prep_mean = sum(prep_ms) / len(prep_ms)
    attn_tops = ops / (attn_mean * 1e-3) / 1e12
    prep_bytes = (
        sage_prep_algorithmic_bytes(b, h, sk, d)
        if sage
        else prep_algorithmic_bytes(b, h, sq, sk, d, workload.is_causal, quantize_query=args.two_step)
    )
    value = ops / (ms_per_step * 1e-3) / 1e12
    log(f"[bench] step {ms_per_step:.4f} ms ({value:.1f} TOPS); attention {attn_mean:.4f} ms "
        f"({attn_tops:.1f} TOPS, {100 * attn_tops / INT8_PEAK_TOPS:.1f}% of INT8 peak); prep {prep_mean:.4f} ms")

    result = {
        "metric": (
            "SageAttention2++ TOPS + % dense INT8/FP8 MFMA peak, 1 MI355X"
            if sage
            else "attention TOPS + % INT8 MFMA peak, B1 H24 S16k D128 fp16, 1 MI355X"
        ),
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded numpy PCG64 per head, fp16 inputs resident in HBM)",
        "config": {
            **workload.as_dict(),
            "operator": args.operator,
            "step": (
                "complete operator call: HIP prep of Q, K, V + fused attention kernel"
                if args.two_step and not sage
                else "complete operator call: HIP prep of K, V + fused attention kernel quantising Q in its prologue"
            ),
            "plan": None,
        },
        "percent_of_int8_peak": round(100 * value / INT8_PEAK_TOPS, 2),
        "attention_kernel": {
            "ms_mean": round(attn_mean, 5),
            "ms_p20_p50_p80": [round(attn_ms[int(f * (len(attn_ms) - 1))], 5) for f in (0.2, 0.5, 0.8)],
            "tops": round(attn_tops, 2),
            "percent_of_int8_peak": round(100 * attn_tops / INT8_PEAK_TOPS, 2),
        },
        "prep": {
            "ms_mean": round(prep_mean, 5),
            "algorithmic_bytes": prep_bytes,
            "gbps": round(prep_bytes / (prep_mean * 1e-3) / 1e9, 1),
            "percent_of_hbm_peak": round(100 * prep_bytes / (prep_mean * 1e-3) / 1e9 / HBM_PEAK_GBPS, 2),
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(attn_tops, 2),
            "peak": INT8_PEAK_TOPS,
            "unit": "TOPS",
            "frac": round(attn_tops / INT8_PEAK_TOPS, 4),
            "traffic": traffic_from_profile(workload.name),
        },
        "cpu_baseline": None,
    }
    from piper_kernels.attention.piper_attention._plan import select_plan

    if sage:
        from piper_kernels.attention.piper_attention._plan import sage_plan

        result["config"]["plan"] = sage_plan(b, h, sq).as_dict()
        result["roofline"]["traffic"] = None
        result["dtype"] = "int8 QK, fp8 e4m3 PV"
    else:
        result["config"]["plan"] = select_plan(b, h, sq, sk, d, workload.is_causal).as_dict()
        result["config"]["qk_granularity"] = args.qk_granularity
    # the sustained dense MFMA rate of this GPU (library probe, after the timed region)
    from piper_kernels._hip import library as native
    from piper_kernels.measure import measure_mfma_peak

    log("[bench] MFMA probe")
    measured = {
        "int8": measure_mfma_peak(native.MFMA_PROBE_I8, device),
        "fp8": measure_mfma_peak(native.MFMA_PROBE_F8, device),
    }
    result["mfma_peak_measured"] = measured
    # how MFMA execution and VALU issue share a SIMD at the attention kernels' occupancy
    from piper_kernels.measure import measure_mfma_valu_sharing

    log("[bench] MFMA/VALU sharing probe")
    result["mfma_valu_sharing"] = measure_mfma_valu_sharing(device)
    result["attention_kernel"]["percent_of_measured_int8_peak"] = round(100 * attn_tops / measured["int8"]["tops"], 2)
    if not args.no_cpu_baseline and not sage:
        log("[bench] cpu baseline")
        result["cpu_baseline"] = cpu_baseline(workload, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

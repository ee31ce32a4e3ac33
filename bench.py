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
region.  Warm-up runs at least ``--warmup`` steps and at least ``--warmup-ms`` of GPU time, so
the clock has ramped before timing starts.

Beside the timing (all after the timed region):

* ``quality``: the timed call's output against FP64 softmax attention on a row slice, next to
  the quantised reference's own distance on the same rows, and against the quantised reference
  (the CPU oracle's output for every head the CPU baseline computed): max and mean absolute
  error, SQNR and cosine (the reference harness's quality columns,
  benchmarks/benchmark_attention.py:249,380), and ``saturation``: how many INT8 Q, K and V
  codes of the call sit at -127 or 127 (the reference harness's saturation fields,
  benchmarks/lib/quality.py:16-41);
* ``cpu_baseline``: the CPU oracle (a numpy restatement of the reference's portable path) on
  whole heads of the same workload (or row ranges of them, where there are fewer heads than
  threads), one task per host thread on all the host threads the run may use, per thread-group
  Q/K scales (the reference's default) and, on one round of tasks, per block;
* ``mfma_peak_measured``: the sustained dense INT8 and FP8 MFMA rate of the same GPU (the
  measurement library's back-to-back MFMA probe, results checked), with the kernel's fraction
  of it in ``attention_kernel``;
* ``issue_sharing``: the measurement library's issue probe (VALU issue per waves per SIMD,
  MFMA/VALU overlap across and within waves, the attention loop's mix with and without its
  MFMAs, LDS bandwidth);
* ``clock``: the engine clock while the workload runs (the measurement library's clock probe on
  a second stream beside ~300 ms of further steps) and the kernel's rate against the INT8 peak
  at that clock;
* ``environment``: GPU, clocks, software versions, host CPU and the source revision.

``schema_version`` numbers this record's layout beyond the driver's fixed keys.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c3] [--no-cpu-baseline] [--two-step]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import subprocess
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path[:0] = [str(REPO), str(REPO / "piper-kernels_amd")]

INT8_PEAK_TOPS = 5033.2  # MI355X dense INT8 MFMA: 256 CU x 2.4 GHz x 8192 ops/clk/CU
HBM_PEAK_GBPS = 8000.0
# The reference's published Piper Attention figures (RTX 5090, BF16 non-causal, p50), by the
# workload of the same shape: benchmarks/README.md:521 (B1 H8 N8192 D128, centred V) and :526
# (B1 H1 N131072 D128, uncentred V, the reference's development control of the same cost)
REFERENCE_R1 = {
    "hardware": "RTX 5090 (SM120), Torch 2.12.1+cu130, Triton 3.7.1",
    "hot_ms": 0.674,
    "hot_tops": 407.8,
    "complete_ms": 0.775,
    "complete_tops": 354.7,
    "sqnr_db_vs_sdpa": 36.08,
    "source": "benchmarks/README.md:521",
}
REFERENCE_R2 = {
    "hardware": "RTX 5090 (SM120), Torch 2.12.1+cu130, Triton 3.7.1",
    "hot_ms": 19.579,
    "hot_tops": 449.3,
    "complete_ms": 19.824,
    "complete_tops": 443.7,
    "sqnr_db_vs_sdpa": 35.48,
    "source": "benchmarks/README.md:526 (uncentred V)",
}
REFERENCE_PUBLISHED = {"r1": REFERENCE_R1, "r2": REFERENCE_R2}
SCHEMA_VERSION = 2  # 2: clock block, quality.saturation, r2


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args() -> argparse.Namespace:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--warmup-ms", type=float, default=300.0, help="minimum GPU time of the warm-up steps")
    parser.add_argument(
        "--workload",
        default="c3",
        choices=["c1", "c2", "c3", "c4", "c5", "r1", "r2"],
        help="BASELINE.json's configurations c1-c5, or r1 / r2: the shapes of the reference's published RTX 5090 "
        "figures (B1 H8 N8192, B1 H1 N131072)",
    )
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--cpu-seconds", type=float, default=15.0, help="target CPU-baseline sample time")
    parser.add_argument("--quality-rows", type=int, default=256, help="query rows per head in the FP64 SDPA check")
    parser.add_argument("--no-probes", action="store_true", help="skip the MFMA-peak and issue probes")
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
    parser.add_argument(
        "--sage-accumulate",
        choices=["fp32", "reference"],
        default="fp32",
        help="SageAttention2++ only: FP32 accumulation across blocks (default) or the reference's FP16 partials",
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


# ---------------------------------------------------------------------------------------
# CPU baseline: the oracle, one (batch, head) slice per worker process and host thread
# ---------------------------------------------------------------------------------------
def _cpu_worker_ready() -> int:
    from threadpoolctl import threadpool_limits

    from oracle import piper_oracle  # noqa: F401  (import before timing)
    from piper_kernels import workloads  # noqa: F401

    threadpool_limits(limits=1)
    return os.getpid()


def _cpu_head(task: tuple[str, int, int, str, int, int]):
    """The full reference computation of query rows [r0, r1) of one (batch, head) slice on one
    thread: K/V means, Q/K/V codes of the whole slice, and the 64-key streaming loop over those
    rows.  Returns the task, its wall time (input generation excluded) and the FP32 output rows."""
    from threadpoolctl import threadpool_limits

    from oracle import piper_oracle as oracle
    from piper_kernels.workloads import WORKLOADS, make_inputs

    name, b, h, granularity, r0, r1 = task
    w = WORKLOADS[name]
    q, k, v = make_inputs(w, heads=[h], batches=[b])
    with threadpool_limits(limits=1):
        start = time.perf_counter()
        prepared = oracle.prepare(q, k, v, w.is_causal, granularity)
        if (r0, r1) != (0, w.query_length):
            prepared = dict(prepared)
            for key in ("query_code", "query_scale"):
                prepared[key] = prepared[key][:, :, r0:r1]
        out = oracle.attention_from_prepared(prepared, w.head_dim**-0.5, w.is_causal, query_offset=r0)
        seconds = time.perf_counter() - start
    return b, h, granularity, r0, r1, seconds, out[0, 0]


def row_range_operations(workload, r0: int, r1: int) -> int:
    """The reference's operation count (4 x pairs x D) for query rows [r0, r1) of one slice; causal
    rows see keys 0..row."""
    pairs = (r1 - r0) * workload.key_length
    if workload.is_causal:
        pairs = (r1 * (r1 + 1) - r0 * (r0 + 1)) // 2
    return 4 * pairs * workload.head_dim


def host_threads() -> int:
    """Host threads the run may use: OMP_NUM_THREADS when set (16 on the GPU box), else the CPU
    count; at most 16, the box's CPU share per GPU."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    threads = int(env) if env.isdigit() and int(env) > 0 else (os.cpu_count() or 1)
    return max(1, min(16, threads))


def _pause(seconds: float) -> int:
    time.sleep(seconds)
    return os.getpid()


def start_cpu_pool(threads: int):
    """Worker processes for the CPU baseline, started before this process touches the GPU (so
    they inherit no GPU state), each with the oracle imported and one numpy thread."""
    import multiprocessing
    from concurrent.futures import ProcessPoolExecutor

    pool = ProcessPoolExecutor(max_workers=threads, mp_context=multiprocessing.get_context("spawn"),
                               initializer=_cpu_worker_ready)
    pids = set(pool.map(_pause, [0.5] * threads))  # every worker started and initialised
    log(f"[bench] cpu baseline: {len(pids)} worker processes ready")
    return pool


def cpu_baseline(pool, threads: int, workload, seconds: float) -> tuple[dict, dict]:
    """Time the CPU oracle on whole (batch, head) slices of the workload, ``threads`` tasks at a
    time in the worker processes (one numpy thread each), until ~``seconds`` of wall time have
    passed or every slice is done; then one round per block.  A workload with fewer slices than
    threads (r2: one head of 131072 rows) splits each slice's query rows into contiguous ranges,
    one task each, so that every thread works and a round stays bounded.  Returns the record and
    the oracle's FP32 outputs of the completed slices by (batch, head)."""
    import numpy as np

    # heads interleaved from both halves (0, H/2, 1, H/2+1, ...) so that a bounded sample covers
    # both of c5's V families (constant along the sequence below H/2, random above)
    half = max(1, workload.heads // 2)
    head_order = sorted(range(workload.heads), key=lambda h: (h % half, h // half))
    slices = [(b, h) for b in range(workload.batch) for h in head_order]
    parts = max(1, threads // len(slices)) if len(slices) < threads else 1
    rows = workload.query_length
    bounds = [(rows * i // parts, rows * (i + 1) // parts) for i in range(parts)]
    tasks = [(b, h, r0, r1) for b, h in slices for r0, r1 in bounds if r1 > r0]
    pieces: dict[tuple[int, int], dict[int, np.ndarray]] = {}
    outputs: dict[tuple[int, int], np.ndarray] = {}
    per_thread_wall = 0.0
    per_thread_ops = 0
    done = 0
    while done < len(tasks) and (done == 0 or per_thread_wall < seconds):
        batch = tasks[done : done + threads]
        start = time.perf_counter()
        for b, h, _, r0, r1, _, out in pool.map(_cpu_head, [(workload.name, b, h, "per_thread", r0, r1)
                                                             for b, h, r0, r1 in batch]):
            pieces.setdefault((b, h), {})[r0] = out
            per_thread_ops += row_range_operations(workload, r0, r1)
            if len(pieces[(b, h)]) == len(bounds):
                outputs[(b, h)] = np.concatenate([pieces[(b, h)][r] for r, _ in bounds])
        per_thread_wall += time.perf_counter() - start
        done += len(batch)
        log(f"[bench] cpu baseline: {done} task(s) per_thread, {per_thread_wall:.1f} s")
    batch = tasks[: min(threads, len(tasks))]
    start = time.perf_counter()
    list(pool.map(_cpu_head, [(workload.name, b, h, "per_warp", r0, r1) for b, h, r0, r1 in batch]))
    warp_wall = time.perf_counter() - start
    warp_ops = sum(row_range_operations(workload, r0, r1) for _, _, r0, r1 in batch)
    log(f"[bench] cpu baseline: {len(batch)} task(s) per_warp, {warp_wall:.1f} s")
    split = f"each slice's {rows} query rows in {parts} contiguous ranges, one task each, " if parts > 1 else ""

    record = {
        "value": per_thread_ops / per_thread_wall / 1e12,
        "unit": "TOPS",
        "cores": threads,
        "kind": "port",
        "per_warp_value": warp_ops / warp_wall / 1e12,
        "sample": (
            f"{workload.name}: {done} of {len(tasks)} tasks over {len(slices)} (batch, head) slices ({split}"
            f"each task the full reference computation: K/V means, per_thread Q/K codes and V codes of its slice, "
            f"64-key streaming loop over its query rows), {threads} at a time in worker processes with one numpy "
            f"thread each; {per_thread_wall:.1f} s wall; per_warp: {len(batch)} tasks in {warp_wall:.1f} s; "
            f"numpy {np.__version__}; "
            f"host threads used {threads} of os.cpu_count={os.cpu_count()}"
        ),
    }
    return record, outputs


# ---------------------------------------------------------------------------------------
# quality
# ---------------------------------------------------------------------------------------
def sdpa_rows_float64(q, k, v, rows: int, scale: float, is_causal: bool):
    """FP64 softmax attention of the first ``rows`` query rows of each [B', H', S, D] slice."""
    import numpy as np

    q64 = q[:, :, :rows].double().cpu().numpy()
    k64 = k.double().cpu().numpy()
    v64 = v.double().cpu().numpy()
    logits = np.matmul(q64, np.swapaxes(k64, -1, -2)) * scale
    if is_causal:
        logits = np.where(np.arange(k64.shape[2])[None, :] > np.arange(rows)[:, None], -np.inf, logits)
    logits -= logits.max(axis=-1, keepdims=True)
    weights = np.exp(logits)
    weights /= weights.sum(axis=-1, keepdims=True)
    return np.matmul(weights, v64)


def quality_block(workload, output, reference_outputs: dict, rows: int) -> dict:
    """The timed call's output against FP64 SDPA (first ``rows`` rows of heads 0 and H/2) and
    against the quantised reference (every slice the CPU baseline computed)."""
    import numpy as np
    import torch

    from piper_kernels.measure import measure_quality
    from piper_kernels.workloads import make_inputs

    def metrics(actual, expected) -> dict:
        m = measure_quality(torch.as_tensor(actual), torch.as_tensor(expected))
        return {"max_abs": m.max_absolute_error, "mean_abs": m.mean_absolute_error, "sqnr_db": round(m.sqnr_db, 2),
                "cosine": m.cosine_similarity}

    heads = sorted({0, workload.heads // 2})  # c5's two V families; the CPU baseline's first slices
    rows = min(rows, workload.query_length)
    q, k, v = make_inputs(workload, batches=[0], heads=heads)
    sdpa = sdpa_rows_float64(q, k, v, rows, workload.head_dim**-0.5, workload.is_causal)
    got = output[:1, heads, :rows].float().cpu().numpy()
    result = {
        "vs_fp64_sdpa": {
            "sample": f"batch 0, heads {heads}, query rows 0..{rows - 1}",
            "output_dtype": str(output.dtype).removeprefix("torch."),
            **metrics(got, sdpa),
        }
    }
    if all((0, h) in reference_outputs for h in heads):
        ref = np.stack([reference_outputs[(0, h)][:rows] for h in heads])[None]
        result["vs_fp64_sdpa"]["reference_fp32"] = metrics(ref, sdpa)
        cast = torch.from_numpy(ref).to(output.dtype).float().numpy()
        result["vs_fp64_sdpa"]["reference_cast_to_output_dtype"] = metrics(cast, sdpa)
    if reference_outputs:
        keys = sorted(reference_outputs)
        actual = torch.stack([output[b, h].float().cpu() for b, h in keys])
        ref32 = torch.stack([torch.from_numpy(reference_outputs[key]) for key in keys])
        result["vs_quantized_reference"] = {
            "sample": f"{len(keys)} whole (batch, head) slices (the CPU baseline's)",
            "fp32_reference": metrics(actual, ref32),
            "reference_cast_to_output_dtype": metrics(actual, ref32.to(output.dtype).float()),
        }
    return result


def saturation_block(q, k, v, scale: float, workload, granularity: str) -> dict:
    """How many INT8 codes of the call's Q, K and V sit at the quantiser's endpoints (-127, 127),
    with the field names of the reference harness's ``QuantizerSaturation``
    (``benchmarks/lib/quality.py:16-41``).  Counted on the GPU from a two-step prep of the timed
    inputs (the fused path never writes query codes), over the valid rows only.  The UINT8
    probability codes exist only inside the attention kernel and are not counted."""
    import torch

    from piper_kernels.attention.piper_attention.hip import _prepare_piper_attention

    b, h, sq, sk, d = workload.shape
    with torch.no_grad():
        prepared = _prepare_piper_attention(q, k, v, scale, workload.is_causal, quantize_query=True,
                                            qk_granularity=granularity)
        keys = torch.arange(prepared.value_code_transposed().shape[2] * 64, device=q.device)
        codes = {
            "query": prepared.query_code[:, :, :sq],
            "key": prepared.key_code()[:, :, :sk],
            # V^T codes [B, H, tiles, D, 64] -> [B, H, D, Sk64], valid keys only
            "value": prepared.value_code_transposed().permute(0, 1, 3, 2, 4).reshape(b, h, d, -1)[..., keys < sk],
        }
        result = {}
        for name, c in codes.items():
            low = int(torch.count_nonzero(c == -127))
            high = int(torch.count_nonzero(c == 127))
            total = c.numel()
            result[name] = {"minimum": -127, "maximum": 127, "minimum_count": low, "maximum_count": high,
                            "count": low + high, "total_count": total, "fraction": (low + high) / total}
    return result


# ---------------------------------------------------------------------------------------
# environment
# ---------------------------------------------------------------------------------------
HIP_ATTRIBUTE_CLOCK_RATE = 5  # hipDeviceAttributeClockRate (hip_runtime_api.h): peak clock in kHz


def peak_sclk_mhz(device) -> int | None:
    """The device's peak engine clock from hipDeviceGetAttribute (torch does not expose it on ROCm),
    called in the HIP runtime this process already has mapped (never a second copy of it)."""
    import ctypes

    try:
        with open("/proc/self/maps") as maps:
            path = next((line.split()[-1] for line in maps if "libamdhip64.so" in line.split()[-1]), None)
        if path is None:
            return None
        hip = ctypes.CDLL(path, mode=os.RTLD_NOLOAD)
    except OSError:
        return None
    value = ctypes.c_int(0)
    if hip.hipDeviceGetAttribute(ctypes.byref(value), HIP_ATTRIBUTE_CLOCK_RATE, int(device.index or 0)) != 0:
        return None
    return value.value // 1000 or None


def source_digest() -> dict:
    """SHA-256 of the measured code as it sits in this tree (the GPU box's copy has no git
    history): the HIP sources and header, the Python package and bench.py, and the built library."""
    import hashlib

    package = REPO / "piper-kernels_amd"
    files = [
        *sorted((package / "csrc").glob("*")),
        *sorted((REPO / "include").glob("*.h")),
        *sorted((package / "piper_kernels").rglob("*.py")),
        *sorted((package / "piper_kernels").rglob("*.json")),
        REPO / "bench.py",
    ]
    digest = hashlib.sha256()
    for path in files:
        if path.is_file():
            digest.update(str(path.relative_to(REPO)).encode() + b"\0" + path.read_bytes())
    library = package / "piper_kernels" / "_hip" / "libpiper_mi355x.so"
    return {
        "sources_sha256": digest.hexdigest(),
        "library_sha256": hashlib.sha256(library.read_bytes()).hexdigest() if library.is_file() else None,
    }


def environment(device) -> dict:
    import numpy as np
    import torch

    props = torch.cuda.get_device_properties(device)
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            cpu = next((line.split(":", 1)[1].strip() for line in f if line.startswith("model name")), cpu)
    except OSError:
        pass
    try:
        revision = subprocess.run(["git", "-C", str(REPO), "rev-parse", "HEAD"], capture_output=True, text=True,
                                  timeout=10).stdout.strip() or None
    except (OSError, subprocess.SubprocessError):
        revision = None
    return {
        "gpu": props.name,
        "arch": props.gcnArchName,
        "compute_units": props.multi_processor_count,
        "max_sclk_mhz": peak_sclk_mhz(device),
        "torch": torch.__version__,
        "hip": torch.version.hip,
        "numpy": np.__version__,
        "python": platform.python_version(),
        "host_cpu": cpu,
        "host_cpu_count": os.cpu_count(),
        "source_revision": revision,
        **source_digest(),
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

    sage = args.operator == "sage_attention_2pp"
    with_cpu_baseline = not args.no_cpu_baseline and not sage
    threads = host_threads()
    pool = start_cpu_pool(threads) if with_cpu_baseline else None  # before any GPU call

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

    if sage:
        from piper_kernels.attention.sage_attention_2pp.hip import _launch_sage_attention_2pp
        from piper_kernels.attention.sage_attention_2pp.hip import _prepare_sage_attention_2pp

        def launch(prepared):
            return _launch_sage_attention_2pp(prepared, accumulate=args.sage_accumulate)

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

    # the timed region's events exist before the warm-up ends, so that no host work (slower under
    # a profiler) leaves the GPU idle, and its clock falling, between warm-up and timing
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    with torch.no_grad():
        # warm-up: at least --warmup steps and at least --warmup-ms of GPU time (the clock ramps)
        warm_steps = 0
        warm_begin = torch.cuda.Event(enable_timing=True)
        warm_begin.record()
        while True:
            for _ in range(max(1, args.warmup) if warm_steps == 0 else 5):
                step()
                warm_steps += 1
            warm_end = torch.cuda.Event(enable_timing=True)
            warm_end.record()
            warm_end.synchronize()
            if warm_steps >= args.warmup and warm_begin.elapsed_time(warm_end) >= args.warmup_ms:
                break
        log(f"[bench] warmup {warm_steps} steps, {warm_begin.elapsed_time(warm_end):.0f} ms")
        log(f"[bench] timing {args.steps} steps")
        torch.cuda.synchronize()
        start = time.perf_counter()
        for i in range(args.steps):
            out = step(events[i])
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - start

        # the engine clock under this load, read on the GPU beside ~300 ms of further steps after the
        # timed region (the clock probe's sleeping waves on a second stream; reads only, the published
        # peak stays the roofline's)
        from piper_kernels.measure import ClockProbe

        probe = ClockProbe(device, duration_ms=300.0)
        for _ in range(5):
            step()  # queue work first, so the probe's waves start beside it
        probe.start()
        guard = time.perf_counter()
        while not probe.done() and time.perf_counter() - guard < 5.0:
            for _ in range(5):
                step()
            torch.cuda.current_stream(device).synchronize()
        clock = probe.summary()

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
        "warmup": warm_steps,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": f"synthetic (seeded numpy PCG64 per head, {workload.as_dict()['dtype']} inputs resident in HBM)",
        # version of this record's layout beyond the driver's fixed keys (as the reference harness's
        # records carry one, benchmarks/lib/reporting.py:18): bump when a field changes meaning
        "schema_version": SCHEMA_VERSION,
        "config": {
            **workload.as_dict(),
            "operator": args.operator,
            **({"sage_accumulate": args.sage_accumulate} if sage else {}),
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
        "quality": None,
    }
    from piper_kernels.attention.piper_attention._plan import select_plan

    if sage:
        from piper_kernels.attention.piper_attention._plan import select_sage_plan

        result["config"]["plan"] = select_sage_plan(b, h, sq, sk, d, workload.is_causal).as_dict()
        result["roofline"]["traffic"] = None
        result["dtype"] = "int8 QK, fp8 e4m3 PV"
    else:
        result["config"]["plan"] = select_plan(b, h, sq, sk, d, workload.is_causal).as_dict()
        result["config"]["qk_granularity"] = args.qk_granularity
        if workload.name in REFERENCE_PUBLISHED:
            # the reference's only published Piper Attention figures are for these shapes, on another
            # GPU (RTX 5090, BF16, p50): the complete call and the hot prepared kernel
            published = REFERENCE_PUBLISHED[workload.name]
            result["vs_baseline"] = round(value / published["complete_tops"], 3)
            result["reference_published"] = {
                **published,
                "kernel_speedup": round(published["hot_ms"] / attn_mean, 3),
                "complete_speedup": round(published["complete_ms"] / ms_per_step, 3),
            }
    result["environment"] = environment(device)
    if clock.get("engine_clock_mhz_median"):
        # the kernel's rate against the dense INT8 peak at the clock it ran at (8192 ops/clk/CU)
        mhz = clock["engine_clock_mhz_median"]
        peak_at_clock = INT8_PEAK_TOPS * mhz / 2400.0
        result["clock"] = {
            **clock,
            "max_sclk_mhz": result["environment"].get("max_sclk_mhz"),
            "window": ("about 300 ms of further steps after the timed region; one sleeping probe wave per XCC "
                       "on a second stream reads the shader clock counter against the wall clock counter"),
            "attention_kernel_cycles_at_median_clock": round(attn_mean * 1e-3 * mhz * 1e6),
            "int8_peak_tops_at_median_clock": round(peak_at_clock, 1),
            "attention_percent_of_int8_peak_at_median_clock": round(100 * attn_tops / peak_at_clock, 2),
        }
    if not args.no_probes:
        # the sustained dense MFMA rate of this GPU and the issue probe (after the timed region)
        from piper_kernels._hip import library as native
        from piper_kernels.measure import measure_issue_sharing, measure_mfma_peak

        log("[bench] MFMA probe")
        measured = {
            "int8": measure_mfma_peak(native.MFMA_PROBE_I8, device),
            "fp8": measure_mfma_peak(native.MFMA_PROBE_F8, device),
        }
        result["mfma_peak_measured"] = measured
        result["attention_kernel"]["percent_of_measured_int8_peak"] = round(
            100 * attn_tops / measured["int8"]["tops"], 2
        )
        log("[bench] issue probe")
        result["issue_sharing"] = measure_issue_sharing(device)
    reference_outputs: dict = {}
    if pool is not None:
        log("[bench] cpu baseline")
        with pool:
            result["cpu_baseline"], reference_outputs = cpu_baseline(pool, threads, workload, args.cpu_seconds)
    if not sage:
        log("[bench] quality")
        result["quality"] = quality_block(workload, out, reference_outputs, args.quality_rows)
        result["quality"]["saturation"] = saturation_block(q, k, v, scale, workload, args.qk_granularity)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

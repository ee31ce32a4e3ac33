"""Focused GPU workloads for rocprofv3 runs (kernel traces and PMC counters).

    python -m piper_kernels.profiling attention --workload c3 --launches 3
        prepare one workload once, then launch only the fused attention kernel (the operator's
        path: the kernel quantises the query itself; --two-step: prepared query codes)
    python -m piper_kernels.profiling attention --workload c3 --plan 16
        the same with launch plan 16 (PIPER_PLAN_* bits; default: the plan select_plan picks)
    python -m piper_kernels.profiling prep --workload c3 --launches 3
        run only the prep pipeline (mean partials, mean finalisation, quantisation; K and V
        only unless --two-step)
    python -m piper_kernels.profiling attention --operator sage_attention_2pp --workload c3
        the same for SageAttention2++ (its K/V prep, then only its attention kernel)
    python -m piper_kernels.profiling copy --bytes 1073741824 --launches 3
        a plain device-to-device copy of a known size: the calibration that turns
        FETCH_SIZE / WRITE_SIZE counter readings into bytes
    python -m piper_kernels.profiling tiles --plan 16
        the fixed cost of a query tile: four non-causal shapes with the same work (B1 H24 D128,
        Sq x Sk = 16384 x 16384, 32768 x 8192, 65536 x 4096, 131072 x 2048; random fp16 inputs)
        timed with HIP events; prints ns per wave-block per SIMD and the least-squares fit
        ns = a + b / n over the n key blocks per tile, whose b / a is the tile's cost in blocks

Run it from the repository root with ``piper-kernels_amd`` on ``sys.path`` (as below), e.g.
``rocprofv3 --pmc FETCH_SIZE --kernel-include-regex attention_kernel -- python -m
piper_kernels.profiling attention --workload c3``.
"""

from __future__ import annotations

import argparse
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("what", choices=["attention", "prep", "copy", "tiles"])
    parser.add_argument("--workload", default="c3")
    parser.add_argument("--launches", type=int, default=3)
    parser.add_argument("--bytes", type=int, default=1 << 30)
    parser.add_argument("--two-step", action="store_true", help="quantise the query in the prep, not the kernel")
    parser.add_argument("--operator", choices=["piper_attention", "sage_attention_2pp"], default="piper_attention")
    parser.add_argument("--plan", type=int, default=None, help="Piper Attention launch plan id (default: the selected plan)")
    args = parser.parse_args(argv)

    import torch

    from piper_kernels.attention.piper_attention.hip import _launch_piper_attention, _prepare_piper_attention
    from piper_kernels.workloads import WORKLOADS, make_inputs

    device = torch.device("cuda", 0)
    if args.what == "copy":
        src = torch.empty(args.bytes // 4, dtype=torch.float32, device=device).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(args.launches):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"copied {args.bytes} bytes x {args.launches}", flush=True)
        return 0
    if args.what == "tiles":
        return tile_cost(device, args.plan)
    w = WORKLOADS[args.workload]
    q, k, v = make_inputs(w, device)
    scale = w.head_dim**-0.5
    fused = not args.two_step
    if args.operator == "sage_attention_2pp":
        from piper_kernels.attention.sage_attention_2pp.hip import (
            _launch_sage_attention_2pp,
            _prepare_sage_attention_2pp,
        )

        with torch.no_grad():
            prepared = _prepare_sage_attention_2pp(q, k, v, scale, w.is_causal)
            for _ in range(args.launches):
                if args.what == "attention":
                    _launch_sage_attention_2pp(prepared)
                else:
                    _prepare_sage_attention_2pp(q, k, v, scale, w.is_causal)
        torch.cuda.synchronize()
        print(f"{args.operator} {args.what} {args.workload} x {args.launches} done", flush=True)
        return 0
    from piper_kernels.attention.piper_attention._plan import MI355XPlan

    plan = None if args.plan is None else MI355XPlan.from_id(args.plan)
    with torch.no_grad():
        prepared = _prepare_piper_attention(q, k, v, scale, w.is_causal, plan=plan, quantize_query=not fused)
        for _ in range(args.launches):
            if args.what == "attention":
                _launch_piper_attention(prepared)
            else:
                _prepare_piper_attention(q, k, v, scale, w.is_causal, quantize_query=not fused)
    torch.cuda.synchronize()
    print(f"{args.what} {args.workload} x {args.launches} done", flush=True)
    return 0


def tile_cost(device, plan_id: int | None) -> int:
    """Equal-work shapes with 256, 128, 64 and 32 key blocks per query tile (see the module doc)."""
    import torch

    from piper_kernels.attention.piper_attention._plan import MI355XPlan
    from piper_kernels.attention.piper_attention.hip import _launch_piper_attention, _prepare_piper_attention

    plan = None if plan_id is None else MI355XPlan.from_id(plan_id)
    gen = torch.Generator(device=device).manual_seed(0)
    points = []
    with torch.no_grad():
        for sq, sk in ((16384, 16384), (32768, 8192), (65536, 4096), (131072, 2048)):
            q, k, v = (torch.randn((1, 24, n, 128), generator=gen, device=device, dtype=torch.float16)
                       for n in (sq, sk, sk))
            prepared = _prepare_piper_attention(q, k, v, 128**-0.5, False, plan=plan, quantize_query=False)
            for _ in range(30):
                _launch_piper_attention(prepared)
            times = []
            for _ in range(5):
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record()
                for _ in range(10):
                    _launch_piper_attention(prepared)
                end.record()
                end.synchronize()
                times.append(start.elapsed_time(end) / 10)
            ms = sorted(times)[2]
            wave_blocks_per_simd = 24 * (sq // 32) * (sk // 64) / 1024
            ns = ms * 1e6 / wave_blocks_per_simd
            points.append((sk // 64, ns))
            print(f"Sq {sq} Sk {sk}: {ms:.4f} ms (median of 5 x 10 launches), {ns:.1f} ns per wave-block per SIMD",
                  flush=True)
            del q, k, v, prepared
    # least squares ns = a + b / n
    xs = [1.0 / n for n, _ in points]
    ys = [ns for _, ns in points]
    mx, my = sum(xs) / len(xs), sum(ys) / len(ys)
    b = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
    a = my - b * mx
    print(f"fit: {a:.1f} ns per wave-block + {b:.1f} ns per tile -> a tile costs {b / a:.2f} wave-blocks beyond its blocks",
          flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

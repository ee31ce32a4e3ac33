"""Offline launch-plan tuner for the MI355X backend (never called at run time).

Counterpart of the reference's ``benchmarks/tune_piper_attention.py:53-221``: a bounded
search over the plan axes the gfx950 kernel exposes (query waves per workgroup and
workgroups per CU, causal
query-tile order -- forward, longest first head by head, or longest first across the heads of
an XCD -- and XCD-aware workgroup order), quality-gated, whose result is frozen into
``mi355x_plans.json`` for ``select_plan``.  With ``--operator sage_attention_2pp`` it tunes the
SageAttention2++ kernel over the same axes (the counterpart of the reference's
``benchmarks/tune_sage_attention_2pp.py``) into ``mi355x_sage_plans.json`` for
``select_sage_plan``; that operator's default plan is three 4-wave workgroups per CU.

    python -m piper_kernels.attention.piper_attention.tune --workloads c1 c2 c3 c4 c5 --write
    python -m piper_kernels.attention.piper_attention.tune --operator sage_attention_2pp --write

For each shape: synthetic inputs are prepared once (K and V; the kernel quantises the query,
as the operator runs it); every candidate plan is launched on the same prepared operands and
gated: its FP32 output must equal the default plan's bit for bit (every plan performs the
same arithmetic per query; only the order of workgroups differs), except Piper Attention's
non-causal key-range split plans (2, 3, 4, 6 or 8 key parts), which merge partial sums in
another order and must stay within 1e-5 (relative to the output's magnitude) of it.  Timing: the GPU first runs
the candidates for ``--warmup-ms`` so the clock has ramped, then ``--rounds`` rounds each
launch every candidate ``--launches`` times back to back, bracketed by HIP events on the
launch stream with no host synchronisation inside a round (the GPU never idles between
candidates), in an order rotated by one each round (no candidate always runs first).  The
fastest passing plan by median is recorded; a plan within ``--margin`` of the default keeps
the default.
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
from dataclasses import replace
from itertools import product
from pathlib import Path

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parents[3]))


SPLIT_PARTS = (2, 3, 4, 6, 8)  # key parts of the split candidates
SPLIT_TOLERANCE = 1e-5  # split plans: max |difference| to the default plan, relative to max(1, max |output|)


def candidate_plans(is_causal: bool, operator: str = "piper_attention"):
    from piper_kernels.attention.piper_attention._plan import MI355XPlan

    # causal orders: (longest first, interleaved across heads); both flags only matter when causal
    orders = ((True, False), (True, True), (False, False)) if is_causal else ((True, False),)
    # occupancy: one 8-wave workgroup, two 4-wave workgroups or three 4-wave workgroups per CU
    occupancy = ((8, False), (4, False), (4, True))
    plans = [
        MI355XPlan(waves=w, causal_longest_first=o, xcd_remap=x, causal_interleave=i, three_per_cu=t)
        for (w, t), (o, i), x in product(occupancy, orders, (True, False))
    ]
    if operator == "piper_attention":
        # work queues per XCC (bit-identical), in each causal order
        plans += [MI355XPlan(waves=4, three_per_cu=True, work_queue=True, causal_longest_first=o, causal_interleave=i)
                  for o, i in orders]
    if operator == "piper_attention" and not is_causal:
        plans += [MI355XPlan(waves=4, three_per_cu=True, key_parts=k, xcd_remap=x)
                  for k, x in product(SPLIT_PARTS, (True, False))]
    return plans


def _operator_entry_points(operator: str):
    """(default plan, prepare(q, k, v, scale, causal, plan), launch(prepared, output=None))."""
    from piper_kernels.attention.piper_attention._plan import MI355XPlan

    if operator == "sage_attention_2pp":
        from piper_kernels.attention.sage_attention_2pp.hip import (
            _launch_sage_attention_2pp,
            _prepare_sage_attention_2pp,
        )

        def prepare(q, k, v, scale, causal, plan):
            return _prepare_sage_attention_2pp(q, k, v, scale, causal, plan=plan)

        return MI355XPlan(waves=4, three_per_cu=True), prepare, _launch_sage_attention_2pp
    from piper_kernels.attention.piper_attention.hip import _launch_piper_attention, _prepare_piper_attention

    def prepare(q, k, v, scale, causal, plan):
        return _prepare_piper_attention(q, k, v, scale, causal, plan=plan, quantize_query=False)

    return MI355XPlan(), prepare, _launch_piper_attention


def tune_shape(q, k, v, is_causal: bool, *, warmup_ms: float, rounds: int, launches: int, margin: float,
               operator: str = "piper_attention") -> dict:
    import torch

    from piper_kernels.attention.piper_attention._plan import shape_key

    b, h, sq, d = q.shape
    sk = k.shape[2]
    default, prepare, launch = _operator_entry_points(operator)
    prepared = prepare(q, k, v, d**-0.5, is_causal, default)
    plans = candidate_plans(is_causal, operator)
    reference = torch.empty(q.shape, device=q.device, dtype=torch.float32)
    launch(prepared, output=reference)
    candidate_out = torch.empty_like(reference)
    bound = SPLIT_TOLERANCE * max(1.0, float(reference.abs().max()))
    passed = {}
    for plan in plans:
        launch(replace(prepared, plan=plan), output=candidate_out)
        torch.cuda.synchronize()
        if plan.key_parts > 1:
            passed[plan] = bool((candidate_out - reference).abs().max() <= bound)
        else:
            passed[plan] = bool(torch.equal(candidate_out, reference))
    times = {plan: [] for plan in plans}
    runs = {plan: replace(prepared, plan=plan) for plan in plans}
    stream = torch.cuda.current_stream()
    warm_start = torch.cuda.Event(enable_timing=True)
    warm_start.record(stream)
    while True:
        for plan in plans:
            launch(runs[plan])
        warm_end = torch.cuda.Event(enable_timing=True)
        warm_end.record(stream)
        warm_end.synchronize()
        if warm_start.elapsed_time(warm_end) >= warmup_ms:
            break
    for r in range(rounds):
        order = plans[r % len(plans) :] + plans[: r % len(plans)]
        events = []
        for plan in order:
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            for _ in range(launches):
                launch(runs[plan])
            end.record(stream)
            events.append((plan, start, end))
        torch.cuda.synchronize()
        for plan, start, end in events:
            times[plan].append(start.elapsed_time(end) / launches)
    medians = {plan: statistics.median(ts) for plan, ts in times.items()}
    best = min((p for p in plans if passed[p]), key=lambda p: medians[p])
    if medians[best] > medians[default] * (1.0 - margin):
        best = default
    batch_heads, ql, kl, hd, causal = shape_key(b, h, sq, sk, d, is_causal)
    return {
        "key": {"batch_heads": batch_heads, "query_length": ql, "key_length": kl, "head_dim": hd, "is_causal": causal},
        "plan": {"waves": best.waves, "causal_longest_first": best.causal_longest_first, "xcd_remap": best.xcd_remap,
                 "causal_interleave": best.causal_interleave, "three_per_cu": best.three_per_cu,
                 **({"key_parts": best.key_parts} if best.key_parts > 1 else {}),
                 **({"work_queue": True} if best.work_queue else {})},
        "candidates": [
            {"plan_id": p.plan_id, **p.as_dict(), "median_ms": round(medians[p], 5),
             ("within_split_tolerance" if p.key_parts > 1 else "bitwise_equal_to_default"): passed[p]}
            for p in plans
        ],
        "default_ms": round(medians[default], 5),
        "chosen_ms": round(medians[best], 5),
    }


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--operator", choices=("piper_attention", "sage_attention_2pp"), default="piper_attention")
    parser.add_argument("--workloads", nargs="+", default=["c1", "c2", "c3", "c4", "c5"])
    parser.add_argument("--warmup-ms", type=float, default=1000.0, help="GPU time of warm-up launches per shape")
    parser.add_argument("--rounds", type=int, default=8)
    parser.add_argument("--launches", type=int, default=3)
    parser.add_argument("--margin", type=float, default=0.01, help="minimum gain over the default plan")
    parser.add_argument("--write", action="store_true", help="write the operator's frozen table next to _plan.py")
    parser.add_argument("--out", type=Path, help="also write the table here")
    args = parser.parse_args(argv)

    import torch

    from piper_kernels.attention.piper_attention._plan import PLAN_TABLE, SAGE_PLAN_TABLE
    from piper_kernels.workloads import WORKLOADS, make_inputs

    device = torch.device("cuda", 0)
    entries = []
    with torch.no_grad():
        for name in args.workloads:
            w = WORKLOADS[name]
            q, k, v = make_inputs(w, device)
            entry = tune_shape(q, k, v, w.is_causal, warmup_ms=args.warmup_ms, rounds=args.rounds,
                               launches=args.launches, margin=args.margin, operator=args.operator)
            entry["workload"] = name
            entries.append(entry)
            print(f"[tune] {name}: default {entry['default_ms']:.4f} ms, chosen {entry['plan']} {entry['chosen_ms']:.4f} ms",
                  file=sys.stderr, flush=True)
            del q, k, v
            torch.cuda.empty_cache()
    table = {
        "operator": args.operator,
        "device": torch.cuda.get_device_properties(device).gcnArchName,
        "tuner": "python -m piper_kernels.attention.piper_attention.tune " + " ".join(argv if argv is not None else sys.argv[1:]),
        "entries": entries,
    }
    text = json.dumps(table, indent=1) + "\n"
    if args.write:
        (SAGE_PLAN_TABLE if args.operator == "sage_attention_2pp" else PLAN_TABLE).write_text(text)
    if args.out:
        args.out.write_text(text)
    print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())

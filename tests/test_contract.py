"""Host-side contract (CPU): validation, target detection, dispatch, plan, custom op, metrics.

Validation cases and messages follow the reference's
tests/attention/piper_attention/test_dispatch.py:98-165; target detection follows
tests/triton/test_targets.py:90-112; metric known answers follow
tests/benchmark_support/test_quality.py:8-22 and test_benchmark_attention.py:349-359.
"""

from __future__ import annotations

import math
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

import piper_kernels
from piper_kernels import piper_attention
from piper_kernels._hip import library as native
from piper_kernels._hip.targets import AcceleratorTarget
from piper_kernels.attention.piper_attention import dispatch
from piper_kernels.attention.piper_attention._plan import MI355XPlan, select_plan
from piper_kernels.measure import (
    attention_operations,
    measure_quality,
    prep_algorithmic_bytes,
    sage_prep_algorithmic_bytes,
)
from piper_kernels.workloads import WORKLOADS, make_inputs

REPO = Path(__file__).resolve().parents[1]


def _inputs():
    q = torch.randn(1, 2, 16, 64, dtype=torch.float16)
    return q, torch.randn_like(q), torch.randn_like(q)


def test_package_root_exports_piper_attention() -> None:
    assert piper_kernels.piper_attention is piper_attention
    assert "piper_attention" in piper_kernels.__all__


@pytest.mark.parametrize("dtype", [torch.float32, torch.int8])
def test_rejects_unsupported_dtype(dtype) -> None:
    q = torch.zeros((1, 1, 8, 64), dtype=dtype)
    with pytest.raises(ValueError, match="float16 or bfloat16"):
        piper_attention(q, q, q)


def test_rejects_non_4d() -> None:
    q = torch.zeros((1, 8, 64), dtype=torch.float16)
    with pytest.raises(ValueError, match=r"shape \[batch, heads, sequence, head_dim\]"):
        piper_attention(q, q, q)


def test_rejects_mismatched_dtypes() -> None:
    q, k, v = _inputs()
    with pytest.raises(ValueError, match="share a dtype"):
        piper_attention(q, k.to(torch.bfloat16), v)


def test_rejects_unequal_heads() -> None:
    q, k, v = _inputs()
    with pytest.raises(ValueError, match="equal batch and head dimensions"):
        piper_attention(q, k[:, :1], v[:, :1])


def test_rejects_unsupported_head_dimension() -> None:
    q = torch.randn(1, 1, 8, 32, dtype=torch.float16)
    with pytest.raises(ValueError, match="head dimensions 64 and 128"):
        piper_attention(q, q, q)


def test_rejects_mismatched_key_value_lengths() -> None:
    q, k, v = _inputs()
    with pytest.raises(ValueError, match="key/value lengths"):
        piper_attention(q, k, v[:, :, :-1])


def test_rejects_rectangular_causal_inputs() -> None:
    q, k, v = _inputs()
    with pytest.raises(ValueError, match="equal query and key lengths"):
        piper_attention(q[:, :, :-1], k, v, is_causal=True)


@pytest.mark.parametrize(("query_length", "key_length"), [(0, 8), (8, 0)])
def test_rejects_empty_sequences(query_length, key_length) -> None:
    q = torch.empty((1, 1, query_length, 64), dtype=torch.float16)
    k = torch.empty((1, 1, key_length, 64), dtype=torch.float16)
    with pytest.raises(ValueError, match="does not accept empty"):
        piper_attention(q, k, k)


def test_rejects_noncontiguous_head_dimension() -> None:
    storage = torch.randn(1, 1, 8, 128, dtype=torch.float16)
    q = storage[..., ::2]
    with pytest.raises(ValueError, match="head dimension must be contiguous"):
        piper_attention(q, q, q)


def test_rejects_autograd() -> None:
    q, k, v = _inputs()
    q.requires_grad_(True)
    with pytest.raises(RuntimeError, match="inference-only"):
        piper_attention(q, k, v)


@pytest.mark.parametrize("scale", [0.0, -1.0, float("inf"), float("nan")])
def test_rejects_invalid_scale(scale) -> None:
    q, k, v = _inputs()
    with pytest.raises(ValueError, match="finite and positive"):
        piper_attention(q, k, v, scale=scale)


def test_cpu_tensors_fail_loudly_instead_of_falling_back() -> None:
    q, k, v = _inputs()
    with pytest.raises(NotImplementedError, match="gfx950"):
        piper_attention(q, k, v)


# ---- target detection ----------------------------------------------------------------
def test_rocm_target_normalises_gcn_arch_name(monkeypatch) -> None:
    monkeypatch.setattr(torch.version, "hip", "7.0.0", raising=False)
    monkeypatch.setattr(
        torch.cuda, "get_device_properties", lambda _d: SimpleNamespace(gcnArchName="gfx950:sramecc+:xnack-")
    )
    target = AcceleratorTarget.from_device(torch.device("cuda", 0))
    assert target == AcceleratorTarget("hip", "gfx950")
    assert target.is_amd_hip and target.supports_piper_mi355x


@pytest.mark.parametrize("arch", ["gfx942", "gfx1201:sramecc+:xnack-", None])
def test_other_amd_architectures_are_not_supported(monkeypatch, arch) -> None:
    monkeypatch.setattr(torch.version, "hip", "7.0.0", raising=False)
    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda _d: SimpleNamespace(gcnArchName=arch))
    assert not AcceleratorTarget.from_device(torch.device("cuda", 0)).supports_piper_mi355x


def test_cpu_and_cuda_targets_are_not_supported(monkeypatch) -> None:
    assert not AcceleratorTarget.from_device(torch.device("cpu")).supports_piper_mi355x
    monkeypatch.setattr(torch.version, "hip", None, raising=False)
    monkeypatch.setattr(torch.cuda, "get_device_capability", lambda _d: (12, 0))
    target = AcceleratorTarget.from_device(torch.device("cuda", 0))
    assert target == AcceleratorTarget("cuda", "sm120") and not target.supports_piper_mi355x


# ---- dispatch ------------------------------------------------------------------------
def test_gfx950_dispatch_routes_to_custom_op_with_default_scale(monkeypatch) -> None:
    calls = []
    monkeypatch.setattr(dispatch.AcceleratorTarget, "from_device", classmethod(lambda cls, d: cls("hip", "gfx950")))
    monkeypatch.setattr(dispatch, "load_library", lambda: None)
    monkeypatch.setattr(dispatch, "hip_piper_attention", lambda q, k, v, s, c: calls.append((s, c)) or q)
    q, k, v = _inputs()
    piper_attention(q, k, v)
    piper_attention(q, k, v, scale=0.2, is_causal=True)
    assert calls == [(64**-0.5, False), (0.2, True)]


def test_gfx950_without_library_raises(monkeypatch, tmp_path) -> None:
    monkeypatch.setattr(dispatch.AcceleratorTarget, "from_device", classmethod(lambda cls, d: cls("hip", "gfx950")))

    def missing():
        return native.load_library(tmp_path / "absent.so")

    monkeypatch.setattr(dispatch, "load_library", missing)
    monkeypatch.setattr(dispatch, "hip_piper_attention", lambda *a: pytest.fail("must not run without library"))
    q, k, v = _inputs()
    with pytest.raises(RuntimeError, match="not built"):
        piper_attention(q, k, v)


def test_every_native_call_runs_under_the_input_device_guard(monkeypatch) -> None:
    """Like the reference's device-guard test (test_dispatch.py:37-96): the prep and the kernel
    launch are issued with the inputs' device current, on that device's current stream.  The
    library is a recording stand-in (layout queries go to the real, host-only function)."""
    from piper_kernels.attention.piper_attention import hip

    real = native.load_library()
    guard = []  # devices of the guards currently entered
    calls = []

    class Guard:
        def __init__(self, device):
            self.device = torch.device(device)

        def __enter__(self):
            guard.append(self.device)

        def __exit__(self, *exc):
            guard.pop()

    class Recorder:
        def prepared_layout(self, shape):
            return real.prepared_layout(shape)

        def prepare(self, args, stream):
            calls.append(("prepare", list(guard), stream, args.flags))

        def attention_forward(self, args, stream):
            calls.append(("attention_forward", list(guard), stream, args.flags))

        def attention_forward_fused(self, args, stream):
            calls.append(("attention_forward_fused", list(guard), stream, args.flags))

    streams = []

    def current_stream(device=None):
        streams.append(torch.device(device))
        return SimpleNamespace(cuda_stream=0x5EED)

    monkeypatch.setattr(native, "load_library", lambda *a: Recorder())
    monkeypatch.setattr(torch.cuda, "device", Guard)
    monkeypatch.setattr(torch.cuda, "current_stream", current_stream)
    monkeypatch.setattr(torch.Tensor, "record_stream", lambda self, stream: None)
    q, k, v = _inputs()
    hip._run_piper_attention(q, k, v, 64**-0.5, False)  # the operator's path: fused query
    hip._run_piper_attention(q, k, v, 64**-0.5, True, fuse_query=False, qk_granularity="per_warp")
    device = q.device
    assert [c[0] for c in calls] == ["prepare", "attention_forward_fused", "prepare", "attention_forward"]
    assert all(c[1] == [device] and c[2] == 0x5EED for c in calls)  # inside exactly the inputs' guard
    assert set(streams) == {device}
    assert calls[0][3] == native.PREPARE_SKIP_QUERY | native.PREPARE_QK_PER_THREAD
    assert calls[1][3] == native.ATTENTION_QK_PER_THREAD
    assert calls[2][3] == 0 and calls[3][3] == 0


# ---- plan ----------------------------------------------------------------------------
def test_plan_selection() -> None:
    from piper_kernels.attention.piper_attention import _plan

    assert _plan.heuristic_plan(1, 24, 16384) == MI355XPlan(waves=8)
    assert _plan.heuristic_plan(1, 2, 193) == MI355XPlan(waves=4)
    # Piper Attention's untuned shapes: three 4-wave workgroups per CU
    for shape in ((1, 24, 16384, False), (1, 24, 16384, True), (2, 32, 8192, False), (2, 40, 32768, False)):
        assert _plan.piper_heuristic_plan(*shape) == MI355XPlan(waves=4, three_per_cu=True)
    # ... with the key range split when the grid is below one round and 256-query tiles leave CUs
    # idle (c1: 64 tiles, 4 parts), or the keys are long and the last round would be ragged
    # (B1 H1 N131072: 1024 tiles = 1.33 rounds, 3 parts = 4 rounds)
    split = lambda parts: MI355XPlan(waves=4, three_per_cu=True, key_parts=parts)  # noqa: E731
    assert _plan.piper_heuristic_plan(1, 8, 1024, False) == split(4)
    assert _plan.piper_heuristic_plan(1, 1, 131072, False, 131072) == split(3)
    assert _plan.piper_heuristic_plan(1, 1, 32768, False) == split(3)
    assert _plan.piper_heuristic_plan(1, 2, 193, False) == split(2)  # 4 key tiles: at most 2 parts
    assert _plan.piper_heuristic_plan(1, 1, 64, False) == MI355XPlan(waves=4, three_per_cu=True)  # one key tile
    assert _plan.piper_heuristic_plan(1, 8, 1024, True) == MI355XPlan(waves=4, three_per_cu=True)  # causal: whole
    assert _plan.split_parts(1, 24, 4096, 4096) == 1 and _plan.split_parts(1, 24, 16384, 16384) == 1
    # ... except non-causal grids of 256-1535 query tiles of 256 rows that cannot fill three
    # 128-row slots per CU: one 8-wave workgroup per CU (r1, B1 H8 N8192, measured)
    assert _plan.piper_heuristic_plan(1, 8, 8192, False) == MI355XPlan(waves=8)
    assert _plan.piper_heuristic_plan(1, 8, 8192, True) == MI355XPlan(waves=4, three_per_cu=True)
    assert _plan.piper_heuristic_plan(1, 24, 4096, False) == MI355XPlan(waves=4, three_per_cu=True)  # 768 tiles
    assert _plan.sage_plan(1, 24, 16384) == MI355XPlan(waves=4, three_per_cu=True)  # SageAttention2++: three per CU
    assert MI355XPlan(8).plan_id == 0 and MI355XPlan(4).plan_id == 1
    assert MI355XPlan(8).as_dict() == {"waves": 8, "causal_longest_first": True, "xcd_remap": True,
                                        "causal_interleave": False, "three_per_cu": False, "key_parts": 1,
                                        "work_queue": False, "block_m": 256, "block_n": 64}
    assert MI355XPlan(4, three_per_cu=True).plan_id == 16 and MI355XPlan(4, three_per_cu=True).block_m == 128
    with pytest.raises(ValueError):
        MI355XPlan(waves=2)
    with pytest.raises(ValueError):
        MI355XPlan(waves=8, three_per_cu=True)
    # the key-range split: three per CU only, 1..8 parts, parts - 1 in bits 5-7
    split = MI355XPlan(4, three_per_cu=True, key_parts=3)
    assert split.plan_id == 16 | (2 << 5) and MI355XPlan.from_id(split.plan_id) == split
    assert split.workgroups(1, 1, 131072) == 3 * 1024
    for bad_parts in (0, 9):
        with pytest.raises(ValueError):
            MI355XPlan(4, three_per_cu=True, key_parts=bad_parts)
    with pytest.raises(ValueError):
        MI355XPlan(8, key_parts=2)
    # the work-queue plan: three per CU, XCD-aware, no split; bit 8
    queue = MI355XPlan(4, three_per_cu=True, work_queue=True)
    assert queue.plan_id == 16 | 256 and MI355XPlan.from_id(272) == queue
    for bad_queue in (dict(waves=8), dict(waves=4), dict(waves=4, three_per_cu=True, key_parts=2),
                      dict(waves=4, three_per_cu=True, xcd_remap=False)):
        with pytest.raises(ValueError):
            MI355XPlan(work_queue=True, **bad_queue)
    for bad in (17, 32, -1, 256, 1 << 5, 16 | 32 | 256, 16 | 4 | 256, 512):
        with pytest.raises(ValueError):
            MI355XPlan.from_id(bad)


def test_plan_ids_round_trip_and_match_the_header() -> None:
    from piper_kernels.attention.piper_attention import _plan

    header = (REPO / "include" / "piper_mi355x.h").read_text()
    for name, value in (("FOUR_WAVES", 1), ("CAUSAL_FORWARD", 2), ("NO_XCD_REMAP", 4), ("CAUSAL_INTERLEAVE", 8),
                        ("THREE_WORKGROUPS", 16), ("WORK_QUEUE", 256), ("MASK", 511)):
        assert f"#define PIPER_PLAN_{name} {value}" in header
    assert "#define PIPER_PLAN_KEY_PARTS(parts) (((parts) - 1) << 5)" in header
    assert "#define PIPER_PLAN_KEY_PARTS_OF(plan) ((((plan) >> 5) & 7) + 1)" in header
    assert (_plan.PLAN_FOUR_WAVES, _plan.PLAN_CAUSAL_FORWARD, _plan.PLAN_NO_XCD_REMAP) == (1, 2, 4)
    assert (_plan.PLAN_CAUSAL_INTERLEAVE, _plan.PLAN_THREE_WORKGROUPS, _plan.PLAN_MASK) == (8, 16, 511)
    assert _plan.PLAN_WORK_QUEUE == 256
    assert _plan.PLAN_KEY_PARTS_SHIFT == 5
    plans = MI355XPlan.all_plans()  # the bit-identical plans
    assert len(set(plans)) == len(plans) == 27 and all(p.key_parts == 1 for p in plans)
    assert sum(p.work_queue for p in plans) == 3
    split = MI355XPlan.split_plans()
    assert len(set(split)) == len(split) == 14 and all(p.three_per_cu and p.key_parts > 1 for p in split)
    for plan in plans + split:
        assert MI355XPlan.from_id(plan.plan_id) == plan


def test_frozen_plan_table_lookup_and_fallback(tmp_path, monkeypatch) -> None:
    import json

    from piper_kernels.attention.piper_attention import _plan

    table = {"entries": [{"key": {"batch_heads": 24, "query_length": 4096, "key_length": 4096, "head_dim": 128,
                                  "is_causal": False},
                          "plan": {"waves": 4, "causal_longest_first": True, "xcd_remap": False}}]}
    path = tmp_path / "plans.json"
    path.write_text(json.dumps(table))
    monkeypatch.setattr(_plan, "PLAN_TABLE", path)
    _plan.frozen_plans.cache_clear()
    try:
        # batch * heads is the key: B2 H12 is the same shape as B1 H24
        assert _plan.select_plan(2, 12, 4096, 4096, 128, False) == MI355XPlan(4, True, False)
        assert _plan.select_plan(1, 24, 4096, 4096, 128, True) == _plan.piper_heuristic_plan(1, 24, 4096, True)
        assert _plan.select_plan(1, 24, 16384, 16384, 128, False) == _plan.piper_heuristic_plan(1, 24, 16384, False)
    finally:
        _plan.frozen_plans.cache_clear()


def test_committed_plan_table_is_well_formed() -> None:
    from piper_kernels.attention.piper_attention import _plan

    _plan.frozen_plans.cache_clear()
    plans = _plan.frozen_plans()
    if not _plan.PLAN_TABLE.exists():
        pytest.skip("no tuned table committed")
    assert plans, "the committed table has no entries"
    for key, plan in plans.items():
        assert len(key) == 5 and isinstance(plan, MI355XPlan)


def test_committed_sage_plan_table_lookup_and_fallback() -> None:
    """SageAttention2++'s frozen table: the tuner's entries are what select_sage_plan returns for
    their shapes (c4 took the interleaved causal order, plan 24), and an untuned shape gets
    sage_plan's three 4-wave workgroups per CU."""
    import json

    from piper_kernels.attention.piper_attention import _plan

    _plan.frozen_sage_plans.cache_clear()
    table = json.loads(_plan.SAGE_PLAN_TABLE.read_text())
    assert table["operator"] == "sage_attention_2pp" and table["entries"]
    for entry in table["entries"]:
        k = entry["key"]
        assert all(c["bitwise_equal_to_default"] for c in entry["candidates"]), entry["workload"]
        chosen = _plan.select_sage_plan(1, k["batch_heads"], k["query_length"], k["key_length"], k["head_dim"],
                                        k["is_causal"])
        assert chosen == MI355XPlan(**entry["plan"])
        assert min(c["median_ms"] for c in entry["candidates"]) >= entry["chosen_ms"] * (1 - 0.01) - 1e-9
    assert _plan.select_sage_plan(4, 32, 8192, 8192, 128, True).plan_id == 24
    assert _plan.select_sage_plan(1, 3, 777, 777, 64, False) == _plan.sage_plan(1, 3, 777)


# ---- custom op -----------------------------------------------------------------------
def test_custom_op_is_registered_with_reference_schema_and_fake() -> None:
    op = torch.ops.piper_kernels.piper_attention.default
    schema = str(op._schema)
    assert "Tensor query, Tensor key, Tensor value, float scale, bool is_causal" in schema
    q = torch.empty((2, 3, 5, 64), dtype=torch.float16, device="meta").transpose(0, 1)
    out = torch.ops.piper_kernels.piper_attention(q, q, q, 0.125, False)
    assert out.device.type == "meta" and out.shape == q.shape and out.is_contiguous()


# ---- measurement ---------------------------------------------------------------------
def test_quality_metrics_have_expected_definitions() -> None:
    reference = torch.tensor([1.0, 2.0, 0.0])
    actual = torch.tensor([1.0, 1.0, 0.0])
    m = measure_quality(actual, reference)
    assert m.mean_absolute_error == pytest.approx(1 / 3)
    assert m.max_absolute_error == 1.0
    assert m.relative_l1_error == pytest.approx(1 / 3)
    assert m.relative_l2_error == pytest.approx(1 / math.sqrt(5))
    assert m.sqnr_db == pytest.approx(10 * math.log10(5))
    assert m.cosine_similarity == pytest.approx(3 / math.sqrt(10))
    assert m.actual_nonfinite_count == m.reference_nonfinite_count == m.nonfinite_mismatch_count == 0


def test_quality_metric_edge_cases() -> None:
    exact = measure_quality(torch.tensor([1.0, -2.0]), torch.tensor([1.0, -2.0]))
    assert exact.max_absolute_error == 0 and math.isinf(exact.sqnr_db) and exact.cosine_similarity == 1.0
    zeros = measure_quality(torch.zeros(3), torch.zeros(3))
    assert zeros.cosine_similarity == 1.0 and math.isnan(zeros.sqnr_db) and zeros.relative_l2_error == 0
    assert measure_quality(torch.zeros(2), torch.ones(2)).cosine_similarity == 0.0
    opposite = measure_quality(torch.tensor([1.0, 2.0]), torch.tensor([-1.0, -2.0]))
    assert opposite.cosine_similarity == -1.0 and opposite.relative_l1_error == pytest.approx(2.0)
    none = measure_quality(torch.tensor([math.nan]), torch.tensor([1.0]))
    assert math.isnan(none.mean_absolute_error) and none.nonfinite_mismatch_count == 1
    # integer and half inputs widen exactly; 64-bit integers are refused; shapes must match
    assert measure_quality(torch.tensor([3], dtype=torch.int8), torch.tensor([1.0], dtype=torch.float16)).max_absolute_error == 2
    with pytest.raises(ValueError, match="64-bit integer"):
        measure_quality(torch.tensor([1]), torch.tensor([1.0]))
    with pytest.raises(ValueError, match="shape mismatch"):
        measure_quality(torch.zeros(2), torch.zeros(3))


def test_quality_counts_nonfinite_values() -> None:
    m = measure_quality(torch.tensor([math.nan, math.inf, 1.0]), torch.tensor([math.nan, 2.0, 1.0]))
    assert m.mean_absolute_error == 0 and math.isinf(m.sqnr_db)
    assert (m.actual_nonfinite_count, m.reference_nonfinite_count, m.nonfinite_mismatch_count) == (2, 1, 1)


def test_effective_operations_account_for_causal_triangle() -> None:
    assert attention_operations(1, 2, 4, 4, 8, False) == 4 * 1 * 2 * 4 * 4 * 8
    assert attention_operations(1, 2, 4, 4, 8, True) == 4 * 1 * 2 * (4 * 5 // 2) * 8
    assert attention_operations(1, 24, 16384, 16384, 128, False) == 3_298_534_883_328


def test_prep_algorithmic_bytes_for_headline_shape() -> None:
    assert prep_algorithmic_bytes(1, 24, 16384, 16384, 128, False) == 454_656_000
    # without the query: fp16 read (2 B), code write (1 B) and one scale per 32 rows of Q drop out
    q_bytes = 3 * 24 * 16384 * 128 + 4 * 24 * 512
    assert prep_algorithmic_bytes(1, 24, 16384, 16384, 128, False, quantize_query=False) == 454_656_000 - q_bytes
    # SageAttention2++: K and V read (2 B) and written (1 B each), K scales per 64 rows, K mean and V scales
    assert sage_prep_algorithmic_bytes(1, 24, 16384, 128) == 6 * 24 * 16384 * 128 + 4 * 24 * (256 + 256)


def test_workload_inputs_are_reproducible_per_head() -> None:
    w = WORKLOADS["c1"]
    q1, k1, v1 = make_inputs(w)
    q2, k2, v2 = make_inputs(w, heads=[3, 5])
    assert q1.shape == (1, 8, 1024, 64) and q1.dtype is torch.float16
    assert torch.equal(q1[:, [3, 5]], q2) and torch.equal(k1[:, [3, 5]], k2) and torch.equal(v1[:, [3, 5]], v2)


def test_reference_benchmark_workload_is_plain_standard_normal() -> None:
    """r1: the shape of the reference's published figures (benchmarks/README.md:521), inputs
    drawn as its benchmark draws them: standard normal Q, K, V with no per-channel offsets."""
    w = WORKLOADS["r1"]
    assert w.shape == (1, 8, 8192, 8192, 128) and w.dtype is torch.bfloat16 and not w.is_causal
    q, k, v = make_inputs(w, heads=[2])
    for x in (q, k, v):
        x = x.float()
        assert abs(x.mean().item()) < 0.01 and abs(x.std().item() - 1.0) < 0.01
        assert x.mean(dim=2).abs().max().item() < 0.05  # no per-channel offset


def test_student_t_workload_has_constant_value_heads() -> None:
    w = WORKLOADS["c5"]
    small = type(w)(**{**w.__dict__, "query_length": 256, "key_length": 256})
    q, k, v = make_inputs(small, heads=[0, 39], batches=[1])
    assert torch.equal(v[0, 0], v[0, 0, :1].expand_as(v[0, 0]))
    assert not torch.equal(v[0, 1], v[0, 1, :1].expand_as(v[0, 1]))


def test_integration_ops_coexist_with_the_reference_registration() -> None:
    """The integration guide's HIP module registers its own qualified op, so it coexists with the
    reference's Triton registration of piper_kernels::piper_attention (triton.py:984), which the
    reference imports on ROCm too (dispatch.py:10-15); a second registration of one name raises."""
    import re
    import subprocess
    import sys

    text = (REPO / "INTEGRATION.md").read_text()
    names = re.findall(r'custom_op\("(piper_kernels::[a-z0-9_]+)"', text)
    assert names and "piper_kernels::piper_attention" not in names
    script = f"""
import torch
SIG = "(Tensor query, Tensor key, Tensor value, float scale, bool is_causal) -> Tensor"
lib = torch.library.Library("piper_kernels", "FRAGMENT")
lib.define("piper_attention" + SIG)   # stand-in for the reference's Triton registration
for name in {names!r}:
    @torch.library.custom_op(name, mutates_args=())
    def op(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scale: float, is_causal: bool) -> torch.Tensor:
        return query.clone()
try:
    lib.define("piper_attention" + SIG)
except RuntimeError:
    print("duplicate registration refused")
print(sorted(n for n in dir(torch.ops.piper_kernels) if n.startswith("piper_attention")))
"""
    result = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=300)
    assert result.returncode == 0, result.stderr
    assert "duplicate registration refused" in result.stdout
    assert "'piper_attention', 'piper_attention_hip'" in result.stdout


"""Parity at the BASELINE.json configurations (c1-c5) on MI355X.

Heads are independent (own means, codes, softmax), so a head subset of a configuration is
that configuration's computation for those heads.  Each case runs at both of the reference's
Q/K granularities: per thread group (the operator's path and the reference portable path's
default, reference.py:42) and per block.  Prep is compared bit for bit on the checked heads
(a prep that also quantises the query); the attention output comes from the operator's path
-- a K/V prep and the fused entry point, whose kernel quantises the query in its prologue --
checked to equal the two-step path bit for bit and compared with the oracle on row slices
(rows are independent; causal slices carry their absolute offset).  Size-independent
properties run on the full shapes: exact preservation of constant-V heads (c5) and causal
independence of future V rows (c4).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _parity import (
    assert_attention_close,
    assert_prep_bit_exact,
    gpu_attention,
    gpu_prepare,
    log,
    oracle_attention,
    prepared_numpy,
)
from oracle import piper_oracle as oracle
from piper_kernels.workloads import WORKLOADS, make_inputs

pytestmark = pytest.mark.gpu

GRANULARITIES = ["per_thread", "per_warp"]


def _row_slice(prep: dict, rows: slice) -> dict:
    sub = dict(prep)
    sub["query_code"] = prep["query_code"][:, :, rows]
    sub["query_scale"] = prep["query_scale"][:, :, rows]
    return sub


def _oracle_rows(prep: dict, rows: slice, scale: float, causal: bool):
    """Oracle output and tie-flip bound of query rows ``rows``."""
    return oracle_attention(_row_slice(prep, rows), scale, causal, query_offset=rows.start)


def _check_heads(name: str, batches: list[int], heads: list[int], row_slices: list[slice], device,
                 granularity: str) -> None:
    w = WORKLOADS[name]
    q, k, v = make_inputs(w, batches=batches, heads=heads)
    scale = w.head_dim**-0.5
    log(f"[case] {name} {granularity} batches={batches} heads={heads} shape={tuple(q.shape)}")
    prep = oracle.prepare(q, k, v, w.is_causal, granularity)
    two_step = gpu_prepare(q, k, v, scale, w.is_causal, device, qk_granularity=granularity)
    assert_prep_bit_exact(prepared_numpy(two_step), prep, two_step.shape, w.is_causal)
    fused = gpu_prepare(q, k, v, scale, w.is_causal, device, quantize_query=False, qk_granularity=granularity)
    out32 = gpu_attention(fused, torch.float32)
    assert torch.equal(out32, gpu_attention(two_step, torch.float32)), "fused and two-step paths differ"
    out32 = out32.cpu().numpy()
    assert np.isfinite(out32).all()
    for rows in row_slices:
        expected, bound = _oracle_rows(prep, rows, scale, w.is_causal)
        assert_attention_close(out32[:, :, rows], expected, f"{name} {granularity} rows {rows.start}:{rows.stop}",
                               flip_bound=bound)


@pytest.mark.parametrize("granularity", GRANULARITIES)
def test_c1_full(gfx950_device, granularity) -> None:
    _check_heads("c1", [0], list(range(8)), [slice(0, 1024)], gfx950_device, granularity)


@pytest.mark.parametrize("granularity", GRANULARITIES)
def test_c2_full_prep_and_row_slices(gfx950_device, granularity) -> None:
    _check_heads("c2", [0], list(range(24)), [slice(0, 256), slice(3840, 4096)], gfx950_device, granularity)


@pytest.mark.parametrize("granularity", GRANULARITIES)
def test_c3_heads(gfx950_device, granularity) -> None:
    _check_heads("c3", [0], [0, 11, 23], [slice(0, 256), slice(8192, 8448), slice(16128, 16384)], gfx950_device,
                 granularity)


@pytest.mark.parametrize("granularity", GRANULARITIES)
def test_c4_causal_heads(gfx950_device, granularity) -> None:
    _check_heads("c4", [0, 3], [0, 31], [slice(0, 256), slice(4000, 4160), slice(7936, 8192)], gfx950_device,
                 granularity)


@pytest.mark.parametrize("granularity", GRANULARITIES)
def test_c5_student_t_heads(gfx950_device, granularity) -> None:
    _check_heads("c5", [0, 1], [0, 19, 20, 39], [slice(0, 128), slice(32640, 32768)], gfx950_device, granularity)


def test_c3_full_shape_runs_and_matches_its_head_subset(gfx950_device) -> None:
    """The full headline shape through the public operator; heads match a separate subset run
    under the same launch plan bit for bit (a one-head grid on its own would take a key-range
    split plan, equal to rounding only)."""
    from piper_kernels import piper_attention
    from piper_kernels.attention.piper_attention._plan import select_plan
    from piper_kernels.attention.piper_attention.hip import _run_piper_attention

    w = WORKLOADS["c3"]
    q, k, v = make_inputs(w, gfx950_device)
    plan = select_plan(*w.shape, w.is_causal)
    assert plan.key_parts == 1
    with torch.no_grad():
        full = piper_attention(q, k, v)
        part = _run_piper_attention(q[:, [5]].contiguous(), k[:, [5]].contiguous(), v[:, [5]].contiguous(),
                                    w.head_dim**-0.5, False, plan=plan)
    torch.cuda.synchronize()
    assert full.shape == q.shape and full.dtype is torch.float16
    assert torch.isfinite(full).all()
    assert torch.equal(full[:, [5]], part)


def test_c5_constant_value_heads_exact_at_full_length(gfx950_device) -> None:
    """c5 heads 0..19 have V constant along the sequence: the output must equal that row exactly."""
    from piper_kernels import piper_attention

    w = WORKLOADS["c5"]
    q, k, v = make_inputs(w, gfx950_device, batches=[0, 1], heads=[0, 7, 19, 20])
    with torch.no_grad():
        out = piper_attention(q, k, v)
    torch.cuda.synchronize()
    for i in range(3):  # heads 0, 7, 19 are constant-V heads
        torch.testing.assert_close(out[:, i], v[:, i], atol=0.0, rtol=0.0)
    assert torch.isfinite(out[:, 3]).all()


def test_c4_future_value_rows_do_not_change_earlier_outputs(gfx950_device) -> None:
    """Causal at full length: replacing V rows >= 4096 leaves rows < 4096 bit-identical."""
    from piper_kernels import piper_attention

    w = WORKLOADS["c4"]
    q, k, v = make_inputs(w, gfx950_device, batches=[1], heads=[3, 17])
    changed = v.clone()
    changed[:, :, 4096:] = torch.randn_like(changed[:, :, 4096:]) * 16
    with torch.no_grad():
        a = piper_attention(q, k, v, is_causal=True)
        b = piper_attention(q, k, changed, is_causal=True)
    torch.cuda.synchronize()
    assert torch.equal(a[:, :, :4096], b[:, :, :4096])
    assert not torch.equal(a[:, :, 4096:], b[:, :, 4096:])


def _sdpa_rows_float64(q, k, v, rows: slice, scale: float, causal: bool) -> np.ndarray:
    """FP64 softmax attention for query rows `rows` (causal rows see keys <= their index)."""
    q64 = oracle.as_float32(q[:, :, rows]).astype(np.float64)
    k64 = oracle.as_float32(k).astype(np.float64)
    v64 = oracle.as_float32(v).astype(np.float64)
    logits = np.matmul(q64, np.swapaxes(k64, -1, -2)) * scale
    if causal:
        query = np.arange(rows.start, rows.stop)[:, None]
        logits = np.where(np.arange(k64.shape[2])[None, :] > query, -np.inf, logits)
    logits -= logits.max(axis=-1, keepdims=True)
    weights = np.exp(logits)
    weights /= weights.sum(axis=-1, keepdims=True)
    return np.matmul(weights, v64)


@pytest.mark.parametrize(
    "name,batches,heads,rows",
    [("c1", [0], list(range(8)), slice(0, 1024)), ("c2", [0], [0, 23], slice(0, 512)),
     ("c3", [0], [0, 17], slice(8000, 8256)), ("c4", [2], [5], slice(7680, 8192)),
     ("c5", [0, 1], [3, 25, 38], slice(20000, 20128))],
    ids=["c1", "c2", "c3", "c4", "c5"],
)
def test_output_against_fp64_sdpa(gfx950_device, name, batches, heads, rows) -> None:
    """The second correctness level of the task statement, against full-precision attention, on
    the operator's path (per-thread-group Q/K scales, the kernel quantising the query).

    Gate: cosine similarity >= 0.9995 against FP64 SDPA (the stated example tolerance), and a
    max-abs error no larger than the quantized reference's own distance to FP64 SDPA plus 2e-3:
    the stated example max-abs (2e-3) is below what the reference algorithm itself reaches
    against SDPA (INT8 Q/K/V and UINT8 P quantisation, largest on c5's Student-t inputs, where
    an outlier sets a whole 32- or 64-row block's scale), so the kernel is held to "no further
    from SDPA than the reference, within the 2e-3 the kernel may differ from the reference".
    """
    w = WORKLOADS[name]
    q, k, v = make_inputs(w, batches=batches, heads=heads)
    scale = w.head_dim**-0.5
    log(f"[case] sdpa envelope {name} batches={batches} heads={heads} rows={rows.start}:{rows.stop}")
    prepared = gpu_prepare(q, k, v, scale, w.is_causal, device=gfx950_device, quantize_query=False,
                           qk_granularity="per_thread")
    got = gpu_attention(prepared, torch.float32).cpu().numpy()[:, :, rows].astype(np.float64)
    expected = _sdpa_rows_float64(q, k, v, rows, scale, w.is_causal)
    reference, _ = _oracle_rows(oracle.prepare(q, k, v, w.is_causal, "per_thread"), rows, scale, w.is_causal)
    reference_err = np.abs(reference.astype(np.float64) - expected)
    err = np.abs(got - expected)
    cosine = (got * expected).sum() / np.sqrt((got * got).sum() * (expected * expected).sum())
    log(f"[quality] {name} vs fp64 sdpa: max {err.max():.3e} (reference {reference_err.max():.3e}) mean {err.mean():.3e} "
        f"(reference {reference_err.mean():.3e}) cos {cosine:.6f}")
    assert cosine >= 0.9995
    assert err.max() <= reference_err.max() + 2e-3

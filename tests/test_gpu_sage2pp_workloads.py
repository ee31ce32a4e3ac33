"""SageAttention2++ parity at the BASELINE.json configurations (c1-c5) on MI355X.

Heads are independent (own K mean, per-channel V scales, codes and softmax), so a head subset
of a configuration is that configuration's computation for those heads.  Prep is compared bit
for bit on the checked heads; the output on row slices against the oracle in the kernel's
arithmetic (rows are independent; causal slices carry their absolute offset).  The full
headline shape runs through the public operator and must reproduce a separate head-subset run
bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _parity import log
from oracle import sage2pp_oracle as oracle
from piper_kernels.workloads import WORKLOADS, make_inputs

pytestmark = pytest.mark.gpu

MEAN_ABS = 1e-4
MAX_ABS = 5e-3


def _bits_equal(a, b) -> bool:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and bool(np.array_equal(a.view(np.uint32), b.view(np.uint32)))


def _check_heads(name: str, batches: list[int], heads: list[int], row_slices: list[slice], device) -> None:
    from piper_kernels.attention.sage_attention_2pp.hip import _launch_sage_attention_2pp, _prepare_sage_attention_2pp

    w = WORKLOADS[name]
    q, k, v = make_inputs(w, batches=batches, heads=heads)
    scale = w.head_dim**-0.5
    log(f"[sage case] {name} batches={batches} heads={heads} shape={tuple(q.shape)}")
    prep = oracle.prepare(q, k, v)
    with torch.no_grad():
        prepared = _prepare_sage_attention_2pp(
            q.to(device), k.to(device), v.to(device), scale, w.is_causal, qk_granularity="per_warp"
        )
        out32 = torch.empty(q.shape, device=device, dtype=torch.float32)
        _launch_sage_attention_2pp(prepared, output=out32)
    torch.cuda.synchronize(device)
    sk = w.key_length
    assert _bits_equal(prepared.key_mean.cpu().numpy(), prep["key_mean"]), "key means differ"
    assert _bits_equal(prepared.key_scale.cpu().numpy(), prep["key_slot_scale"]), "key scales differ"
    assert _bits_equal(prepared.value_scale.cpu().numpy(), prep["value_scale"]), "value scales differ"
    assert np.array_equal(prepared.key_code().cpu().numpy()[:, :, :sk], prep["key_code"]), "key codes differ"
    assert np.array_equal(prepared.value_code().cpu().numpy()[:, :, :sk], prep["value_code"]), "value codes differ"
    out = out32.cpu().numpy()
    assert np.isfinite(out).all()
    for rows in row_slices:
        sub = dict(prep)
        sub["query_code"] = prep["query_code"][:, :, rows]
        sub["query_scale"] = prep["query_scale"][:, :, rows]
        expected = oracle.attention_from_prepared(sub, scale, w.is_causal, accumulate="fp32", query_offset=rows.start)
        err = np.abs(out[:, :, rows] - expected)
        log(f"   rows {rows.start}:{rows.stop}: mean {err.mean():.2e} max {err.max():.2e}")
        assert err.mean() <= MEAN_ABS and err.max() <= MAX_ABS, (rows, err.mean(), err.max())


def test_c1(gfx950_device) -> None:
    _check_heads("c1", [0], list(range(8)), [slice(0, 1024)], gfx950_device)


def test_c2_row_slices(gfx950_device) -> None:
    _check_heads("c2", [0], list(range(24)), [slice(0, 256), slice(3840, 4096)], gfx950_device)


def test_c3_heads(gfx950_device) -> None:
    _check_heads("c3", [0], [0, 11, 23], [slice(0, 256), slice(8192, 8448), slice(16128, 16384)], gfx950_device)


def test_c4_causal_heads(gfx950_device) -> None:
    _check_heads("c4", [0, 3], [0, 31], [slice(0, 256), slice(4000, 4160), slice(7936, 8192)], gfx950_device)


def test_c5_student_t_heads(gfx950_device) -> None:
    _check_heads("c5", [0, 1], [0, 19, 20, 39], [slice(0, 128), slice(32640, 32768)], gfx950_device)


def test_c3_full_shape_matches_its_head_subset(gfx950_device) -> None:
    from piper_kernels import sage_attention_2pp

    w = WORKLOADS["c3"]
    q, k, v = make_inputs(w, gfx950_device)
    with torch.no_grad():
        full = sage_attention_2pp(q, k, v)
        part = sage_attention_2pp(q[:, [5]].contiguous(), k[:, [5]].contiguous(), v[:, [5]].contiguous())
    torch.cuda.synchronize()
    assert full.shape == q.shape and full.dtype is torch.float16
    assert torch.isfinite(full).all()
    assert torch.equal(full[:, [5]], part)

"""piper_prepare_static (no caller workspace: the mean partials live in the library's static
per-GPU scratch) against piper_prepare, through the C ABI on MI355X: every prepared byte the
header specifies and the attention output equal, on two calls in a row, the second smaller."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _parity import gpu_attention, log, prepared_numpy

pytestmark = pytest.mark.gpu

CASES = [
    # (B, H, Sq, Sk, D, dtype, causal): the second is smaller and reuses the scratch the first filled
    (1, 4, 4096, 4096, 128, torch.float16, False),
    (1, 2, 300, 193, 64, torch.bfloat16, False),
]


def _inputs(case, seed):
    b, h, sq, sk, d, dtype, _ = case
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((b, h, sq, d), generator=g).to(dtype)
    k = (torch.randn((b, h, sk, d), generator=g) + torch.randn((b, h, 1, d), generator=g)).to(dtype)
    v = (torch.randn((b, h, sk, d), generator=g) + 2 * torch.randn((b, h, 1, d), generator=g)).to(dtype)
    return q, k, v


def _prepare(q, k, v, d, causal, device, static):
    from piper_kernels.attention.piper_attention.hip import _prepare_piper_attention

    with torch.no_grad():
        prepared = _prepare_piper_attention(
            q.to(device), k.to(device), v.to(device), d**-0.5, causal, static_workspace=static
        )
    torch.cuda.synchronize(device)
    return prepared


def test_static_scratch_prep_equals_workspace_prep(gfx950_device) -> None:
    for i, case in enumerate(CASES):
        b, h, sq, sk, d, dtype, causal = case
        log(f"[case] piper_prepare_static call {i + 1}: {case}")
        q, k, v = _inputs(case, 700 + i)
        static = _prepare(q, k, v, d, causal, gfx950_device, static=True)
        reference = _prepare(q, k, v, d, causal, gfx950_device, static=False)
        got, expected = prepared_numpy(static), prepared_numpy(reference)
        for name, value in expected.items():
            if value is None:
                assert got[name] is None, name
                continue
            a = np.ascontiguousarray(got[name])
            e = np.ascontiguousarray(value)
            assert a.shape == e.shape and a.dtype == e.dtype, name
            assert np.array_equal(a.view(np.uint8), e.view(np.uint8)), f"{name} differs (call {i + 1})"
        out_static = gpu_attention(static, torch.float32)
        out_reference = gpu_attention(reference, torch.float32)
        assert torch.equal(out_static, out_reference), f"attention output differs (call {i + 1})"

"""Behavioural invariants of the HIP path (the reference's GPU suite, test_triton.py:212-376)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _parity import gpu_attention, gpu_prepare, log
from oracle import piper_oracle as oracle
from piper_kernels.attention.piper_attention._plan import MI355XPlan

pytestmark = pytest.mark.gpu


def test_centered_value_restores_constant_value_exactly(gfx950_device) -> None:
    """test_triton.py:212-222: constant V comes back bit-exact through the fused path."""
    from piper_kernels import piper_attention

    torch.manual_seed(56)
    for dtype in (torch.bfloat16, torch.float16):
        q = torch.randn(1, 2, 1024, 128, dtype=dtype, device=gfx950_device)
        k = torch.randn_like(q)
        row = torch.randn(1, 2, 1, 128, dtype=dtype, device=gfx950_device)
        v = row.expand_as(q).contiguous()
        with torch.no_grad():
            out = piper_attention(q, k, v)
        torch.testing.assert_close(out, v, atol=0.0, rtol=0.0)


def test_causal_output_is_independent_of_future_value_rows(gfx950_device) -> None:
    """test_triton.py:225-242: rows < 32 do not see V rows >= 32, bit for bit."""
    from piper_kernels import piper_attention

    torch.manual_seed(62)
    q = torch.randn(1, 1, 65, 64, dtype=torch.float16, device=gfx950_device)
    k = torch.randn_like(q)
    v = torch.randn_like(q)
    changed = v.clone()
    changed[:, :, 32:] = torch.randn_like(changed[:, :, 32:]) * 32
    with torch.no_grad():
        a = piper_attention(q, k, v, is_causal=True)
        b = piper_attention(q, k, changed, is_causal=True)
    torch.testing.assert_close(a[:, :, :32], b[:, :, :32], atol=0.0, rtol=0.0)


def test_large_value_scale_stays_finite(gfx950_device) -> None:
    """test_triton.py:245-266: a V row of 40000 keeps the multipliers and output finite."""
    q = torch.ones((1, 1, 64, 64), dtype=torch.float16)
    k = torch.ones_like(q)
    k[:, :, 0] = -1
    v = torch.ones_like(q)
    v[:, :, 0] = 40000
    prepared = gpu_prepare(q, k, v, 64**-0.5, False, gfx950_device)
    out = gpu_attention(prepared, torch.float16)
    assert torch.isfinite(prepared.value_inv_multiplier()).all()
    assert torch.isfinite(out).all()


def test_biased_value_quality_against_sdpa(gfx950_device) -> None:
    """test_triton.py:269-282: linspace(-8, 8) feature offsets, MSE vs SDPA < 1e-3."""
    from piper_kernels import piper_attention

    torch.manual_seed(57)
    q = torch.randn(1, 1, 1024, 128, dtype=torch.bfloat16)
    k = torch.randn_like(q)
    offset = torch.linspace(-8, 8, 128).reshape(1, 1, 1, 128)
    v = (offset + torch.randn_like(q.float()) * 0.25).to(torch.bfloat16)
    with torch.no_grad():
        actual = piper_attention(q.to(gfx950_device), k.to(gfx950_device), v.to(gfx950_device))
    expected = oracle.sdpa_float64(q, k, v)
    mse = float(np.mean((actual.float().cpu().numpy() - expected) ** 2))
    log(f"[quality] biased V mse vs fp64 sdpa = {mse:.3e}")
    assert mse < 1e-3


def test_plans_and_repeated_runs_are_bitwise_identical(gfx950_device) -> None:
    """Each query wave computes independently: every launch plan and a rerun agree exactly."""
    torch.manual_seed(61)
    q = torch.randn(1, 2, 700, 128, dtype=torch.bfloat16)
    k = torch.randn_like(q)
    v = torch.randn_like(q)
    outs = []
    for plan in MI355XPlan.all_plans() + [MI355XPlan()]:
        prepared = gpu_prepare(q, k, v, 128**-0.5, True, gfx950_device, plan=plan)
        outs.append(gpu_attention(prepared, torch.float32).cpu())
    assert all(torch.equal(outs[0], o) for o in outs[1:])


def test_torch_compile_fullgraph_on_permuted_inputs(gfx950_device) -> None:
    """test_triton.py:356-376: the custom op traces under torch.compile(fullgraph=True)."""
    from piper_kernels import piper_attention

    torch.manual_seed(60)
    qs = torch.randn(3, 2, 128, 64, device=gfx950_device, dtype=torch.float16)
    ks = torch.randn_like(qs)
    vs = torch.randn_like(qs)
    q, k, v = (t.permute(1, 0, 2, 3) for t in (qs, ks, vs))

    def consumer(q, k, v):
        return -piper_attention(q, k, v)

    with torch.no_grad():
        expected = consumer(q, k, v)
        actual = torch.compile(consumer, fullgraph=True)(q, k, v)
    assert torch.equal(actual, expected)


def test_strided_inputs_match_contiguous(gfx950_device) -> None:
    """Any [B,H,S,D] view with a contiguous head dim is read in place and gives the same bits."""
    from piper_kernels import piper_attention

    torch.manual_seed(63)
    base = torch.randn(1, 100, 3, 4, 128, dtype=torch.float16, device=gfx950_device)  # [B,S,3,H,D]
    q, k, v = (base[:, :, i].transpose(1, 2) for i in range(3))  # [B,H,S,D] views
    with torch.no_grad():
        strided = piper_attention(q, k, v)
        dense = piper_attention(q.contiguous(), k.contiguous(), v.contiguous())
    assert torch.equal(strided, dense)

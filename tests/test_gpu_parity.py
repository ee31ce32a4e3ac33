"""GPU parity of the HIP path with the CPU oracle: bit-exact prep, tolerance attention.

Mirrors the reference's GPU suite (tests/attention/piper_attention/test_triton.py) on
MI355X: the HIP path is compared with the oracle at the same Q/K granularity, as
test_triton.py:35-36 compares its backend with the reference.  Both of the reference's
granularities run: per thread group ("per_thread", the portable path's default and the
operator's) and per block ("per_warp", its grouped SM12x Triton path).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _parity import (
    GOLDEN,
    assert_attention_close,
    assert_prep_bit_exact,
    gpu_attention,
    gpu_prepare,
    load_golden,
    log,
    oracle_attention,
    prepared_numpy,
)
from oracle import piper_oracle as oracle
from piper_kernels.attention.piper_attention._plan import MI355XPlan

pytestmark = pytest.mark.gpu

FIXTURES = sorted(GOLDEN.glob("*.npz"))


@pytest.mark.parametrize("fixture", FIXTURES, ids=[p.stem for p in FIXTURES])
def test_prep_is_bit_exact_with_golden_fixture(fixture, gfx950_device) -> None:
    g = load_golden(fixture)
    log(f"[case] prep golden {fixture.stem} shape={tuple(g['query'].shape)}/{tuple(g['key'].shape)}")
    prepared = gpu_prepare(g["query"], g["key"], g["value"], g["scale"], g["is_causal"], gfx950_device)
    expected = {
        "query_code": g["query_code"],
        "query_block_scale": g["query_block_scale"],
        "key_code": g["key_code"],
        "key_block_scale": g["key_block_scale"],
        "key_mean": g["key_mean"],
        "value_code": g["value_code"],
        "value_scale": g["value_scale"],
        "value_mean": g["value_mean"],
    }
    assert_prep_bit_exact(prepared_numpy(prepared), expected, prepared.shape, g["is_causal"])


@pytest.mark.parametrize("fixture", FIXTURES, ids=[p.stem for p in FIXTURES])
@pytest.mark.parametrize(
    "plan", [MI355XPlan(waves=8), MI355XPlan(waves=4), MI355XPlan(waves=4, three_per_cu=True)], ids=["w8", "w4", "w3"]
)
def test_attention_matches_golden_fixture(fixture, plan, gfx950_device) -> None:
    g = load_golden(fixture)
    log(f"[case] attention golden {fixture.stem} plan={plan.plan_id}")
    prepared = gpu_prepare(g["query"], g["key"], g["value"], g["scale"], g["is_causal"], gfx950_device, plan=plan)
    out32 = gpu_attention(prepared, torch.float32).cpu().numpy()
    expected, bound = oracle_attention(oracle.prepare(g["query"], g["key"], g["value"], g["is_causal"], "per_warp"),
                                       g["scale"], g["is_causal"])
    np.testing.assert_array_equal(expected, g["output_per_warp"])  # the fixture is the oracle's output
    assert_attention_close(out32, g["output_per_warp"], f"{fixture.stem} fp32", flip_bound=bound)
    # the output in the input dtype is the FP32 result rounded to nearest even
    out = gpu_attention(prepared, prepared.output.dtype).float().cpu().numpy()
    np.testing.assert_array_equal(out, oracle.cast_output(out32, str(g["dtype"])))


SHAPES = [
    # (B, H, Sq, Sk, D, dtype, causal)
    (1, 2, 1, 1, 64, torch.float16, False),
    (1, 1, 31, 33, 128, torch.float16, False),
    (1, 2, 64, 64, 128, torch.bfloat16, False),
    (2, 1, 127, 65, 64, torch.bfloat16, False),
    (1, 2, 193, 193, 128, torch.float16, False),
    (1, 2, 193, 193, 64, torch.float16, True),
    (1, 1, 300, 300, 128, torch.bfloat16, True),
    (1, 3, 257, 1000, 128, torch.float16, False),
    (1, 1, 1000, 257, 64, torch.bfloat16, False),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(str(x) for x in s[:5]) + f"-{s[5]}-c{int(s[6])}")
def test_random_shapes_match_oracle(shape, gfx950_device) -> None:
    b, h, sq, sk, d, dtype, causal = shape
    log(f"[case] random {shape}")
    g = torch.Generator().manual_seed(1000 + sq + sk + d)
    q = torch.randn((b, h, sq, d), generator=g).to(dtype)
    k = (torch.randn((b, h, sk, d), generator=g) + torch.randn((b, h, 1, d), generator=g)).to(dtype)
    v = (torch.randn((b, h, sk, d), generator=g) + 2 * torch.randn((b, h, 1, d), generator=g)).to(dtype)
    scale = d**-0.5
    prep = oracle.prepare(q, k, v, causal, "per_warp")
    prepared = gpu_prepare(q, k, v, scale, causal, gfx950_device)
    assert_prep_bit_exact(prepared_numpy(prepared), prep, prepared.shape, causal)
    expected, bound = oracle_attention(prep, scale, causal)
    out32 = gpu_attention(prepared, torch.float32).cpu().numpy()
    assert_attention_close(out32, expected, f"random {shape}", flip_bound=bound)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(str(x) for x in s[:5]) + f"-{s[5]}-c{int(s[6])}")
def test_per_thread_granularity_matches_oracle(shape, gfx950_device) -> None:
    """The reference portable path's default Q/K granularity (reference.py:42, "per_thread":
    sage/reference.py:23-58): codes and every thread-group scale bit for bit, the output within
    the same tolerance, against the oracle's per_thread restatement."""
    b, h, sq, sk, d, dtype, causal = shape
    log(f"[case] per_thread {shape}")
    g = torch.Generator().manual_seed(2000 + sq + sk + d)
    # every thread group gets its own magnitude, so a scale read from the wrong group shows:
    # query row r scaled by 1 + 4 (r % 8) / 7 (group r % 8: 1x to 5x), key row r by
    # 1 + 4 ((r % 8) // 2) / 3 (group (r % 8) // 2: 1x to 5x)
    q_rows = 1 + 4 * (torch.arange(sq) % 8).reshape(1, 1, sq, 1) / 7
    k_rows = 1 + 4 * (torch.arange(sk) % 8 // 2).reshape(1, 1, sk, 1) / 3
    q = (torch.randn((b, h, sq, d), generator=g) * q_rows).to(dtype)
    k = (torch.randn((b, h, sk, d), generator=g) * k_rows + torch.randn((b, h, 1, d), generator=g)).to(dtype)
    v = (torch.randn((b, h, sk, d), generator=g) + 2 * torch.randn((b, h, 1, d), generator=g)).to(dtype)
    scale = d**-0.5
    prep = oracle.prepare(q, k, v, causal, "per_thread")
    prepared = gpu_prepare(q, k, v, scale, causal, gfx950_device, qk_granularity="per_thread")
    assert_prep_bit_exact(prepared_numpy(prepared), prep, prepared.shape, causal)
    expected, bound = oracle_attention(prep, scale, causal)
    out32 = gpu_attention(prepared, torch.float32).cpu().numpy()
    assert_attention_close(out32, expected, f"per_thread {shape}", flip_bound=bound)
    # the fused entry point quantises the query per thread group in its prologue, bit-identically
    fused = gpu_prepare(q, k, v, scale, causal, gfx950_device, quantize_query=False, qk_granularity="per_thread")
    assert torch.equal(gpu_attention(fused, torch.float32).cpu(), torch.from_numpy(out32))


@pytest.mark.parametrize("fixture", FIXTURES, ids=[p.stem for p in FIXTURES])
def test_per_thread_output_matches_golden_fixture(fixture, gfx950_device) -> None:
    g = load_golden(fixture)
    log(f"[case] per_thread golden {fixture.stem}")
    prepared = gpu_prepare(
        g["query"], g["key"], g["value"], g["scale"], g["is_causal"], gfx950_device, quantize_query=False,
        qk_granularity="per_thread",
    )
    out32 = gpu_attention(prepared, torch.float32).cpu().numpy()
    expected, bound = oracle_attention(oracle.prepare(g["query"], g["key"], g["value"], g["is_causal"], "per_thread"),
                                       g["scale"], g["is_causal"])
    np.testing.assert_array_equal(expected, g["output_per_thread"])
    assert_attention_close(out32, g["output_per_thread"], f"{fixture.stem} per_thread", flip_bound=bound)


MEAN_CASES = [
    # (workload, batches, heads): head subsets of the c1-c5 benchmark workloads at their full S
    ("c2", None, [0, 7, 23]),
    ("c3", None, [0, 23]),
    ("c4", [0, 3], [0, 31]),
    ("c5", [1], [0, 39]),
]


@pytest.mark.parametrize("case", MEAN_CASES, ids=[c[0] for c in MEAN_CASES])
def test_means_are_the_reference_torch_cpu_means(case, gfx950_device) -> None:
    """The HIP prep's K and V means equal, bit for bit, what the reference itself computes on
    CPU -- key.float().mean(dim=2) (sage/reference.py:88-89) and value.float().mean(dim=2)
    (reference.py:47-51) -- at the workloads' full sequence lengths (16 to 32768 keys)."""
    from piper_kernels.workloads import WORKLOADS, make_inputs

    name, batches, heads = case
    w = WORKLOADS[name]
    q, k, v = make_inputs(w, batches=batches, heads=heads)
    log(f"[case] means {name} batches={batches} heads={heads} S={w.key_length}")
    prepared = gpu_prepare(q, k, v, w.head_dim**-0.5, w.is_causal, gfx950_device)
    got = prepared_numpy(prepared)
    key_mean = k.float().mean(dim=2).numpy()
    assert np.array_equal(got["key_mean"].view(np.uint32), key_mean.view(np.uint32))
    if w.is_causal:
        assert not got["value_mean"].any()
    else:
        value_mean = v.float().mean(dim=2).numpy()
        assert np.array_equal(got["value_mean"].view(np.uint32), value_mean.view(np.uint32))


def test_public_operator_runs_custom_op_and_keeps_dtype(gfx950_device) -> None:
    from piper_kernels import piper_attention

    torch.manual_seed(54)
    for dtype in (torch.float16, torch.bfloat16):
        q = torch.randn(1, 2, 193, 128, dtype=dtype)
        k = torch.randn_like(q)
        v = torch.randn_like(q)
        with torch.no_grad():
            actual = piper_attention(q.to(gfx950_device), k.to(gfx950_device), v.to(gfx950_device))
        # the operator quantises Q/K per thread group, like the reference's portable path
        expected = oracle.piper_attention_reference(q, k, v, None, False, "per_thread")
        assert actual.dtype is dtype and actual.shape == q.shape and actual.is_contiguous()
        error = np.abs(actual.float().cpu().numpy() - expected)
        log(f"[parity] public op {dtype}: mean={error.mean():.3e} max={error.max():.3e}")
        # the reference's own envelope for its optimised backend (test_triton.py:139-145)
        assert error.mean() < 0.003 and error.max() < 0.12


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_extreme_block_maxima_take_the_subtracting_path(causal, gfx950_device) -> None:
    """The kernel forms P codes from E = exp2(x) and C = 2^(log2 255 - block max) while every
    block maximum of the wave lies within +-96 (log2 units), and subtracts the maximum before
    exp2 otherwise.  Query rows scaled 40x give block maxima of several hundred; rows left at
    N(0, 1) stay in range, so waves of both kinds, and mixed blocks, meet the oracle's gate."""
    torch.manual_seed(31)
    b, h, s, d = 1, 2, 512, 128
    q = torch.randn(b, h, s, d)
    q[:, :, 64:192] *= 40.0  # two and a half waves of large logits
    q[:, :, 300:301] *= 40.0  # one large row inside an otherwise ordinary wave
    q = q.to(torch.float16)
    k = (torch.randn(b, h, s, d) + torch.randn(b, h, 1, d)).to(torch.float16)
    v = (torch.randn(b, h, s, d) + 2 * torch.randn(b, h, 1, d)).to(torch.float16)
    scale = d**-0.5
    log(f"[case] extreme block maxima causal={causal}")
    prep = oracle.prepare(q, k, v, causal, "per_thread")
    prepared = gpu_prepare(q, k, v, scale, causal, gfx950_device, quantize_query=False, qk_granularity="per_thread")
    out32 = gpu_attention(prepared, torch.float32).cpu().numpy()
    expected, bound = oracle_attention(prep, scale, causal)
    assert_attention_close(out32, expected, f"extreme maxima causal={causal}", flip_bound=bound)

"""Pins of the CPU oracle (runs on CPU, no GPU).

Each oracle function is checked against something that does not restate it: exact
rational arithmetic, hand-derived index tables, the reference's own bounds and envelopes,
an independent FP64 non-streaming evaluation, closed forms, and library routines.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import fp64_check
from oracle import piper_oracle as oracle


# --------------------------------------------------------------------------------------
# exact-arithmetic helpers (independent of numpy's float32 arithmetic)
# --------------------------------------------------------------------------------------
def fraction_to_float32(value: Fraction) -> float:
    """Round an exact rational to the nearest float32 (ties to even), for normal results."""
    if value == 0:
        return 0.0
    sign = -1 if value < 0 else 1
    value = abs(value)
    exponent = value.numerator.bit_length() - value.denominator.bit_length()
    if Fraction(2) ** exponent > value:
        exponent -= 1
    # value in [2^e, 2^(e+1)): 24 significant bits -> unit 2^(e-23)
    unit = Fraction(2) ** (exponent - 23)
    scaled = value / unit
    floor = scaled.numerator // scaled.denominator
    rest = scaled - floor
    if rest > Fraction(1, 2) or (rest == Fraction(1, 2) and floor % 2 == 1):
        floor += 1
    return float(sign * floor * unit)


def round_half_even(value: Fraction) -> int:
    return round(value)  # Fraction.__round__ rounds half to even


def exact_scale(amax: float) -> float:
    """amax / 127 + 1e-7 with IEEE float32 roundings, derived with exact rationals."""
    quotient = fraction_to_float32(Fraction(amax) / 127)
    return fraction_to_float32(Fraction(quotient) + Fraction(float(np.float32(1e-7))))


def exact_code(x: float, scale: float) -> int:
    q = fraction_to_float32(Fraction(x) / Fraction(scale))
    return max(-127, min(127, round_half_even(Fraction(q))))


# --------------------------------------------------------------------------------------
# sequence mean
# --------------------------------------------------------------------------------------
def _torch_mean_bits(x: torch.Tensor, threads: int) -> np.ndarray:
    """The reference's call (reference.py:50, sage/reference.py:89) on CPU, as FP32 bits."""
    previous = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        return x.float().mean(dim=2).numpy().view(np.uint32)
    finally:
        torch.set_num_threads(previous)


@pytest.mark.parametrize("length", [1, 5, 15, 16, 17, 64, 255, 256, 257, 1000, 4095, 4096, 4097, 8192, 12289])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_sequence_mean_is_torch_cpu_mean_bit_for_bit(length: int, dtype: torch.dtype) -> None:
    g = torch.Generator().manual_seed(length)
    # head dims are multiples of 32 (the operator accepts 64 and 128): torch's CPU kernel runs
    # its vectorised cascade on every column of such widths
    x = (torch.randn((1, 2, length, 64), generator=g) * 3 + torch.randn((1, 2, 1, 64), generator=g) * 5).to(dtype)
    got = oracle.sequence_mean(oracle.as_float32(x)).view(np.uint32)
    for threads in (1, 4):
        assert np.array_equal(got, _torch_mean_bits(x, threads))


def test_sequence_mean_is_torch_cpu_mean_on_a_permuted_view() -> None:
    # [B, S, H, D] memory viewed as [B, H, S, D]: torch reduces the same rows in the same order
    g = torch.Generator().manual_seed(11)
    x = (torch.randn((2, 3000, 3, 64), generator=g) * 2 + 0.5).to(torch.float16).permute(0, 2, 1, 3)
    assert np.array_equal(oracle.sequence_mean(oracle.as_float32(x)).view(np.uint32), _torch_mean_bits(x, 4))


def test_sequence_mean_is_torch_cpu_mean_where_the_order_matters() -> None:
    # huge and tiny values (bf16 range): every regrouping of the additions changes the result
    x = np.ones((1, 1, 9000, 32), dtype=np.float32)
    x[0, 0, 0, 0] = 2.0**100
    x[0, 0, 4095, 1] = -(2.0**100)
    x[0, 0, 300:310, 2] = 2.0**30
    x[0, 0, 8191, 2] = -(2.0**31)
    x[0, 0, 0, 5] = 2.0**30  # absorbs the ones of its first blocks, not of the exact sum
    t = torch.from_numpy(x).to(torch.bfloat16)
    got = oracle.sequence_mean(oracle.as_float32(t)).view(np.uint32)
    assert np.array_equal(got, _torch_mean_bits(t, 1))
    exact = (oracle.as_float32(t).astype(np.float64).sum(axis=2) / 9000).astype(np.float32).view(np.uint32)
    assert not np.array_equal(got, exact)  # the case really distinguishes the orders


def test_sequence_mean_uses_longer_blocks_past_2_pow_19_rows() -> None:
    assert [oracle.cascade_block_rows(n) for n in (1, 16, 2**16, 2**19, 2**19 + 1, 2**24)] == [16] * 4 + [32, 64]
    g = torch.Generator().manual_seed(3)
    x = (torch.randn((1, 1, 2**19 + 37, 32), generator=g) * 4).to(torch.float16)
    assert np.array_equal(oracle.sequence_mean(oracle.as_float32(x)).view(np.uint32), _torch_mean_bits(x, 1))


def test_sequence_mean_of_negative_zeros_is_positive_zero() -> None:
    x = np.full((1, 1, 70, 32), -0.0, dtype=np.float32)
    mean = oracle.sequence_mean(x)
    assert not np.signbit(mean).any()
    assert np.array_equal(mean.view(np.uint32), _torch_mean_bits(torch.from_numpy(x), 1))


# --------------------------------------------------------------------------------------
# quantisers
# --------------------------------------------------------------------------------------
def test_per_block_codes_and_scales_match_exact_derivation() -> None:
    g = torch.Generator().manual_seed(7)
    x = (torch.randn((1, 1, 40, 8), generator=g) * 2).to(torch.float16)
    x32 = oracle.as_float32(x)
    codes, scales = oracle.quantize_per_group(x32, 32)
    assert codes.shape == (1, 1, 40, 8) and scales.shape == (1, 1, 2)
    for block in range(2):
        rows = x32[0, 0, block * 32 : (block + 1) * 32]
        scale = exact_scale(float(np.abs(rows).max()))
        assert float(scales[0, 0, block]) == scale
        for r in range(rows.shape[0]):
            for d in range(8):
                assert codes[0, 0, block * 32 + r, d] == exact_code(float(rows[r, d]), scale)


def test_rounding_is_half_to_even_at_exact_ties() -> None:
    # amax = 127 * s exactly representable: x / s lands on exact half integers
    scale = np.float32(1.0)
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 126.5, 200.0, -200.0], dtype=np.float32)
    assert oracle._codes(x, scale).tolist() == [0, 2, 2, 0, -2, 126, 127, -127]


def test_per_thread_query_groups_are_rows_t_t8_t16_t24() -> None:
    rows = np.arange(64, dtype=np.float32) + 1  # row r has magnitude r + 1
    q = np.broadcast_to(rows[None, None, :, None], (1, 1, 64, 8)).copy()
    _, scale = oracle.quantize_query_per_thread(q)
    for block in range(2):
        for t in range(8):
            group_max = max(block * 32 + t + 8 * i + 1 for i in range(4))
            for i in range(4):
                assert float(scale[0, 0, block * 32 + 8 * i + t]) == exact_scale(float(group_max))


def test_per_thread_key_groups_are_rows_8a_2t_c() -> None:
    rows = np.arange(64, dtype=np.float32) + 1
    k = np.broadcast_to(rows[None, None, :, None], (1, 1, 64, 8)).copy()
    _, scale = oracle.quantize_key_per_thread(k)
    for t in range(4):
        group = [8 * a + 2 * t + c for a in range(8) for c in range(2)]
        group_max = max(group) + 1
        for row in group:
            assert float(scale[0, 0, row]) == exact_scale(float(group_max))


def test_group_scale_slots_are_the_per_row_scales_of_each_thread_group() -> None:
    """query_group_scales_per_thread / key_group_scales_per_thread (the slots the HIP prep stores)
    against a direct loop over each zero-padded block's thread groups, and against the per-row
    scales of quantize_*_per_thread (pinned by the interleave tables above), on ragged lengths."""
    rng = np.random.default_rng(71)
    for length in (1, 31, 33, 64, 95, 130):
        x = (rng.standard_normal((1, 2, length, 16)) * rng.uniform(0.1, 8.0, (1, 2, length, 1))).astype(np.float32)
        q_slots = oracle.query_group_scales_per_thread(x)
        k_slots = oracle.key_group_scales_per_thread(x)
        assert q_slots.shape == (1, 2, -(-length // 32), 8) and k_slots.shape == (1, 2, -(-length // 64), 4)
        for h in range(2):
            for block in range(q_slots.shape[2]):
                for t in range(8):
                    rows = [32 * block + t + 8 * i for i in range(4)]
                    amax = max((float(np.abs(x[0, h, r]).max()) for r in rows if r < length), default=0.0)
                    assert float(q_slots[0, h, block, t]) == exact_scale(amax)
            for block in range(k_slots.shape[2]):
                for t in range(4):
                    rows = [64 * block + 8 * a + 2 * t + c for a in range(8) for c in range(2)]
                    amax = max((float(np.abs(x[0, h, r]).max()) for r in rows if r < length), default=0.0)
                    assert float(k_slots[0, h, block, t]) == exact_scale(amax)
        _, q_rows = oracle.quantize_query_per_thread(x)
        _, k_rows = oracle.quantize_key_per_thread(x)
        r = np.arange(length)
        assert np.array_equal(q_rows, q_slots[:, :, r // 32, r % 8])
        assert np.array_equal(k_rows, k_slots[:, :, r // 64, (r % 8) // 2])


@pytest.mark.parametrize("is_causal", [False, True])
def test_tie_flip_bound_covers_codes_rounded_the_other_way(is_causal: bool) -> None:
    """attention_from_prepared's flip bound: rounding every near-tie probability code the other
    way (a planted rounding difference) moves each row by no more than the bound, and rows with
    no near-tie code are unchanged."""
    torch.manual_seed(72)
    q = torch.randn(1, 2, 96, 64, dtype=torch.float16)
    k = torch.randn(1, 2, 96, 64, dtype=torch.float16) * 2
    v = torch.randn(1, 2, 96, 64, dtype=torch.float16) + 3
    prep = oracle.prepare(q, k, v, is_causal, "per_thread")
    scale = 64**-0.5
    exact = oracle.attention_from_prepared(prep, scale, is_causal)
    for window in (1e-5, 2e-2):
        out, bound = oracle.attention_from_prepared(prep, scale, is_causal, tie_window=window)
        assert np.array_equal(out, exact) and bound.shape == exact.shape[:3] and (bound >= 0).all()
        flipped, same_bound = oracle.attention_from_prepared(prep, scale, is_causal, tie_window=window, flip_ties=True)
        assert np.array_equal(same_bound, bound)
        moved = np.abs(flipped.astype(np.float64) - exact).max(axis=-1)
        assert (moved <= bound * (1 + 1e-5) + 1e-6).all()
        assert not moved[bound == 0].any()
    # the wide window catches many codes, and flipping them does move the output
    assert (bound > 0).mean() > 0.5 and moved.max() > 1e-3


@pytest.mark.parametrize("granularity", ["per_thread", "per_warp"])
def test_quantize_query_key_bound_and_centering(granularity: str) -> None:
    """tests/attention/test_qk_quantization.py:10-33 of the reference."""
    torch.manual_seed(70)
    q = torch.randn(2, 3, 35, 64, dtype=torch.float16)
    k = torch.randn(2, 3, 67, 64, dtype=torch.float16)
    r = oracle.quantize_query_key(oracle.as_float32(q), oracle.as_float32(k), granularity)
    k_centered = oracle.as_float32(k) - oracle.sequence_mean(oracle.as_float32(k))[:, :, None, :]
    q_err = np.abs(r["query_code"].astype(np.float32) * r["query_scale"][..., None] - oracle.as_float32(q))
    k_err = np.abs(r["key_code"].astype(np.float32) * r["key_scale"][..., None] - k_centered)
    assert r["query_code"].shape == q.shape and r["key_code"].shape == k.shape
    assert r["query_scale"].shape == q.shape[:3] and r["key_scale"].shape == k.shape[:3]
    assert (q_err <= r["query_scale"][..., None] / 2 + 1e-6).all()
    assert (k_err <= r["key_scale"][..., None] / 2 + 1e-6).all()


def test_unknown_granularity_raises() -> None:
    x = np.zeros((1, 1, 8, 64), dtype=np.float32)
    with pytest.raises(ValueError, match="unknown Q/K quantization granularity"):
        oracle.quantize_query_key(x, x, "row")


def test_value_codes_match_exact_derivation() -> None:
    g = torch.Generator().manual_seed(9)
    v = (torch.randn((1, 1, 6, 16), generator=g) * 5).to(torch.bfloat16)
    v32 = oracle.as_float32(v)
    codes, scales = oracle.quantize_value_per_key(v32)
    for row in range(6):
        scale = exact_scale(float(np.abs(v32[0, 0, row]).max()))
        assert float(scales[0, 0, row]) == scale
        assert codes[0, 0, row].tolist() == [exact_code(float(x), scale) for x in v32[0, 0, row]]


# --------------------------------------------------------------------------------------
# attention recurrence
# --------------------------------------------------------------------------------------
def _inputs(b, h, sq, sk, d, dtype, seed, v_bias=2.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((b, h, sq, d), generator=g).to(dtype)
    k = (torch.randn((b, h, sk, d), generator=g) + torch.randn((b, h, 1, d), generator=g)).to(dtype)
    v = (torch.randn((b, h, sk, d), generator=g) + v_bias * torch.randn((b, h, 1, d), generator=g)).to(dtype)
    return q, k, v


@pytest.mark.parametrize(
    "case",
    [
        (1, 2, 70, 70, 64, torch.float16, False),
        (1, 1, 130, 130, 128, torch.bfloat16, True),
        (2, 1, 33, 200, 64, torch.float16, False),
        (1, 1, 200, 129, 128, torch.bfloat16, False),
    ],
)
def test_streaming_oracle_matches_fp64_closed_form(case) -> None:
    b, h, sq, sk, d, dtype, causal = case
    q, k, v = _inputs(b, h, sq, sk, d, dtype, seed=sq + sk)
    for granularity in ("per_warp", "per_thread"):
        prep = oracle.prepare(q, k, v, causal, granularity)
        streaming = oracle.attention_from_prepared(prep, d**-0.5, causal)
        closed = fp64_check.attention_fp64(prep, d**-0.5, causal)
        err = np.abs(streaming - closed)
        assert err.mean() < 1e-5 and err.max() < 1e-2, (err.mean(), err.max())


def test_zero_query_single_tile_matches_closed_form() -> None:
    _, k, v = _inputs(1, 1, 5, 50, 64, torch.float16, seed=3)
    q = torch.zeros((1, 1, 5, 64), dtype=torch.float16)
    prep = oracle.prepare(q, k, v, False, "per_warp")
    out = oracle.attention_from_prepared(prep, 0.125, False)
    expected = fp64_check.single_tile_zero_query(
        prep["value_code"][0, 0], prep["value_scale"][0, 0], prep["value_mean"][0, 0]
    )
    np.testing.assert_allclose(out[0, 0], np.broadcast_to(expected, out[0, 0].shape), rtol=1e-5, atol=1e-5)


def test_single_key_returns_its_value() -> None:
    q, k, v = _inputs(1, 2, 3, 1, 64, torch.float16, seed=4)
    out = oracle.piper_attention_reference(q, k, v, None, False, "per_warp")
    np.testing.assert_array_equal(oracle.cast_output(out, "float16"), oracle.as_float32(v).repeat(3, axis=2))


@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_oracle_is_close_to_exact_attention(head_dim: int, is_causal: bool) -> None:
    """tests/attention/piper_attention/test_reference.py:9-39 of the reference."""
    torch.manual_seed(51)
    q = torch.randn(1, 2, 65, head_dim, dtype=torch.bfloat16)
    k = torch.randn_like(q)
    v = torch.randn_like(q)
    actual = oracle.cast_output(oracle.piper_attention_reference(q, k, v, head_dim**-0.5, is_causal), "bfloat16")
    expected = oracle.sdpa_float64(q, k, v, is_causal=is_causal)
    error = np.abs(actual - expected)
    assert np.isfinite(actual).all()
    assert error.mean() < 0.01 and error.max() < 0.2


def test_oracle_restores_constant_value_exactly() -> None:
    """test_reference.py:42-57."""
    torch.manual_seed(52)
    q = torch.randn(1, 2, 65, 64, dtype=torch.float16)
    k = torch.randn_like(q)
    v = torch.randn(1, 2, 1, 64, dtype=torch.float16).expand_as(q).contiguous()
    for granularity in ("per_thread", "per_warp"):
        out = oracle.piper_attention_reference(q, k, v, 64**-0.5, False, granularity)
        np.testing.assert_array_equal(oracle.cast_output(out, "float16"), oracle.as_float32(v))


def test_causal_oracle_is_independent_of_future_value_rows() -> None:
    """test_reference.py:60-76."""
    torch.manual_seed(53)
    q = torch.randn(1, 1, 65, 64, dtype=torch.float16)
    k = torch.randn_like(q)
    v = torch.randn_like(q)
    changed = v.clone()
    changed[:, :, 32:] = torch.randn_like(changed[:, :, 32:]) * 32
    a = oracle.piper_attention_reference(q, k, v, 64**-0.5, True)
    b = oracle.piper_attention_reference(q, k, changed, 64**-0.5, True)
    np.testing.assert_array_equal(a[:, :, :32], b[:, :, :32])


def test_rectangular_call_with_explicit_scale() -> None:
    """test_dispatch.py:18-34: Sq=9, Skv=11, scale=0.2."""
    torch.manual_seed(50)
    q = torch.randn(1, 1, 9, 64, dtype=torch.float16)
    k = torch.randn(1, 1, 11, 64, dtype=torch.float16)
    v = torch.randn_like(k)
    out = oracle.piper_attention_reference(q, k, v, 0.2, False)
    assert out.shape == (1, 1, 9, 64) and np.isfinite(out).all()


def test_query_offset_reproduces_causal_rows_of_the_full_call() -> None:
    q, k, v = _inputs(1, 1, 150, 150, 64, torch.float16, seed=8)
    prep = oracle.prepare(q, k, v, True, "per_warp")
    full = oracle.attention_from_prepared(prep, 0.125, True)
    sub = dict(prep)
    sub["query_code"] = prep["query_code"][:, :, 100:130]
    sub["query_scale"] = prep["query_scale"][:, :, 100:130]
    part = oracle.attention_from_prepared(sub, 0.125, True, query_offset=100)
    np.testing.assert_array_equal(part, full[:, :, 100:130])


def test_bfloat16_rounding_is_round_to_nearest_even() -> None:
    x = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.0e38, np.inf], dtype=np.float32)
    expected = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(oracle.cast_output(x, "bfloat16"), expected)

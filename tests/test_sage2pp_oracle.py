"""Pinning the SageAttention2++ oracle (oracle/sage2pp_oracle.py) on the CPU.

* the E4M3 codec against torch's ``float8_e4m3fn`` cast, bit for bit;
* the per-channel V quantisation against the reference's torch expression
  (``sage_attention_2pp/reference.py:22-25``) evaluated by torch, bit for bit;
* the recurrence, with its two roundings switched off, against an FP64 softmax over the
  dequantised operands; a single key against its closed form; the reference's SDPA envelope
  (``tests/attention/sage_attention_2pp/test_reference.py:12-35``);
* the size of the difference between the reference's FP16 partials and the FP32
  accumulation the MI355X kernel performs, which sets the GPU tests' tolerance.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import piper_oracle
from oracle import sage2pp_oracle as oracle


def _torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_decode_matches_torch_on_every_code() -> None:
    codes = np.arange(256, dtype=np.uint8)
    expected = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = oracle.fp8_e4m3_decode(codes)
    both_nan = np.isnan(expected) & np.isnan(got)
    assert np.array_equal(got[~both_nan], expected[~both_nan])
    assert np.array_equal(np.isnan(got), np.isnan(expected))
    assert got[0x7E] == 448.0 and got[0x01] == 2.0**-9 and got[0x08] == 2.0**-6


def test_e4m3_encode_matches_torch_cast() -> None:
    rng = np.random.default_rng(0)
    finite = oracle.fp8_e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float32)  # 0 .. 448
    mids = ((finite[:-1].astype(np.float64) + finite[1:]) / 2).astype(np.float32)
    neighbours = np.concatenate([np.nextafter(mids, np.float32(1e9)), np.nextafter(mids, np.float32(0))])
    edges = np.array([448.00003, 448.5, 463.99, 464.0, 464.01, 470.0, 480.0, 1e4, 1e30, np.inf,
                      2.0**-10, 3 * 2.0**-11, 2.0**-12, 1e-30, 0.0], dtype=np.float32)
    wide = rng.uniform(-460, 460, 20000).astype(np.float32)
    small = (rng.uniform(-1, 1, 20000) * 2.0 ** rng.integers(-14, 3, 20000)).astype(np.float32)
    x = np.concatenate([finite, mids, neighbours, edges, wide, small])
    x = np.concatenate([x, -x])
    assert np.array_equal(oracle.fp8_e4m3_encode(x), _torch_e4m3(x))


def test_value_quantization_matches_reference_expression() -> None:
    torch.manual_seed(1)
    for dtype in (torch.float16, torch.bfloat16):
        v = torch.randn(2, 3, 100, 64, dtype=dtype) * 3
        v[0, 1, :, 5] = 0  # an all-zero channel: scale 1e-7, codes 0
        # reference.py:22-25, evaluated by torch
        scale_t = v.float().abs().amax(dim=2) / 2.25 + 1e-7
        codes_t = (v.float() / scale_t[:, :, None, :]).to(torch.float8_e4m3fn).view(torch.uint8)
        codes, scale = oracle.quantize_value_per_channel(piper_oracle.as_float32(v))
        assert np.array_equal(scale, scale_t.numpy())
        assert np.array_equal(codes, codes_t.numpy())
        assert np.abs(oracle.fp8_e4m3_decode(codes)).max() <= 2.25


def _dequantised_softmax(prep: dict, scale: float, is_causal: bool) -> np.ndarray:
    """Independent FP64 evaluation: softmax(S * qs * ks * scale) @ (v8 * vs), not streamed."""
    q = prep["query_code"].astype(np.float64)
    k = prep["key_code"].astype(np.float64)
    logits = np.einsum("bhqd,bhkd->bhqk", q, k)
    logits *= prep["query_scale"][..., :, None].astype(np.float64) * prep["key_scale"][..., None, :] * scale
    if is_causal:
        sq, sk = logits.shape[-2:]
        logits = np.where(np.arange(sk)[None, :] > np.arange(sq)[:, None], -np.inf, logits)
    w = np.exp(logits - logits.max(axis=-1, keepdims=True))
    w /= w.sum(axis=-1, keepdims=True)
    v = oracle.fp8_e4m3_decode(prep["value_code"]).astype(np.float64) * prep["value_scale"][:, :, None, :]
    return np.einsum("bhqk,bhkd->bhqd", w, v)


@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("shape", [(1, 2, 65, 64), (1, 1, 200, 128), (2, 1, 130, 64)])
def test_recurrence_without_rounding_is_exact_softmax(shape, is_causal) -> None:
    rng = np.random.default_rng(2)
    q, k, v = (rng.standard_normal(shape).astype(np.float16) for _ in range(3))
    prep = oracle.prepare(q, k, v)
    d = shape[-1]
    got = oracle.attention_from_prepared(prep, d**-0.5, is_causal, accumulate="fp32", quantize_probabilities=False)
    expected = _dequantised_softmax(prep, d**-0.5, is_causal)
    # FP32 exp and sums over up to 200 keys
    np.testing.assert_allclose(got, expected, rtol=2e-5, atol=2e-6)
    # the reference mode differs only by its FP16 partials: relative 2**-11 per block
    got_ref = oracle.attention_from_prepared(prep, d**-0.5, is_causal, quantize_probabilities=False)
    assert np.abs(got_ref - expected).max() < 4e-3


def test_single_key_closed_form() -> None:
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 1, 5, 64)).astype(np.float16)
    k = rng.standard_normal((1, 1, 1, 64)).astype(np.float16)
    v = rng.standard_normal((1, 1, 1, 64)).astype(np.float16)
    prep = oracle.prepare(q, k, v)
    for mode in oracle.ACCUMULATE_MODES:
        got = oracle.attention_from_prepared(prep, 0.125, False, accumulate=mode)
        # one key: p = exp(ln 448) in FP32, its E4M3 value is 448 exactly
        p = np.exp(oracle.P_FP8_LN_MAX)
        v8 = oracle.fp8_e4m3_decode(prep["value_code"][0, 0, 0]).astype(np.float32)
        partial = np.float32(448.0) * v8
        if mode == "reference":
            partial = partial.astype(np.float16).astype(np.float32)
        expected = partial * prep["value_scale"][0, 0] / p
        np.testing.assert_allclose(got[0, 0], np.broadcast_to(expected, got[0, 0].shape), rtol=2e-7, atol=0)


@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_reference_envelope_against_sdpa(dtype, head_dim, is_causal) -> None:
    """tests/attention/sage_attention_2pp/test_reference.py:12-35 (mean < 0.01, max < 0.2)."""
    torch.manual_seed(41)
    query = torch.randn(1, 2, 65, head_dim, dtype=dtype)
    key = torch.randn_like(query)
    value = torch.randn_like(query)
    actual = piper_oracle.cast_output(
        oracle.sage_attention_2pp_reference(query, key, value, head_dim**-0.5, is_causal), str(dtype).removeprefix("torch.")
    )
    expected = piper_oracle.sdpa_float64(query, key, value, head_dim**-0.5, is_causal)
    error = np.abs(actual - expected)
    assert np.isfinite(actual).all()
    assert error.mean() < 0.01 and error.max() < 0.2


def test_fp32_accumulation_stays_close_to_fp16_partials() -> None:
    """The MI355X kernel's arithmetic (FP32 accumulation, V scale at the end) against the
    reference's FP16 partials: this bounds what the GPU tests may see beyond exp/summation
    rounding."""
    rng = np.random.default_rng(4)
    for shape, causal in (((1, 2, 193, 128), False), ((1, 2, 193, 64), True), ((1, 1, 1024, 128), False)):
        q, k, v = (rng.standard_normal(shape).astype(np.float16) for _ in range(3))
        prep = oracle.prepare(q, k, v)
        ref = oracle.attention_from_prepared(prep, shape[-1] ** -0.5, causal)
        fp32 = oracle.attention_from_prepared(prep, shape[-1] ** -0.5, causal, accumulate="fp32")
        diff = np.abs(ref - fp32)
        assert diff.mean() < 2e-4 and diff.max() < 2e-3, (shape, diff.mean(), diff.max())


def test_unknown_accumulation_mode_raises() -> None:
    prep = oracle.prepare(*(np.zeros((1, 1, 4, 64), np.float16),) * 3)
    with pytest.raises(ValueError, match="accumulation mode"):
        oracle.attention_from_prepared(prep, 0.125, False, accumulate="bf16")

"""CPU oracle for SageAttention2++'s forward pass (numpy restatement).

TEST INFRASTRUCTURE ONLY.  This module is the checker: it may be imported by
``tests/``, by ``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg of
``bench.py``, and by nothing else.  The product path (the ``piper_kernels``
package and its HIP library) never imports, calls or links it.

It restates the portable PyTorch reference of ``jumbledpoophj/piper-kernels`` 0.2.1,
``src/piper_kernels/attention/sage_attention_2pp/reference.py:15-104``:

* K smoothing and INT8 Q/K codes, shared with Piper Attention
  (:func:`oracle.piper_oracle.quantize_query_key`), at either of the reference's
  granularities (the ``granularity`` argument): ``per_thread`` -- per thread group, the
  default of the reference's portable path (``reference.py:35``) and of the MI355X operator
  and smoke test -- or ``per_warp`` -- one scale per 32 query rows and per 64 key rows, the
  grouped scales of the reference's SM12x Triton path (``sage_attention_2pp/_policy.py:63``)
  that its GPU test compares against (``tests/attention/sage_attention_2pp/test_triton.py:33-34``);
  the functions here default to ``per_warp``, the granularity the golden fixtures were made at;
* per-channel FP8 E4M3 V codes, ``scale = amax_S|v| / 2.25 + 1e-7`` (``reference.py:22-25``);
* the 64-key online-softmax loop whose frame is shifted by ln(448) so probabilities land
  in FP8's range, FP8 probabilities, and 64-key partial products rounded to FP16
  (``reference.py:58-104``).

The K mean is :func:`oracle.piper_oracle.sequence_mean`, torch's CPU FP32 summation order
(the reference's ``key_float.mean(dim=2)``), shared with Piper Attention.

``accumulate="fp32"`` restates the MI355X kernel's arithmetic instead of the reference's
FP16 partials: gfx950's FP8 MFMA accumulates in FP32, so the kernel keeps one FP32
accumulator across all key blocks (rescaled when the running maximum moves) and applies
the per-channel V scale once in the epilogue.  The difference between the two modes is the
reference's model of NVIDIA's FP16-accumulating MMA (``reference.py:95-98``).

Parity status (tests/test_sage2pp_oracle.py):

* :func:`fp8_e4m3_encode` / :func:`fp8_e4m3_decode` -- pinned against torch's own
  ``float8_e4m3fn`` cast on every code, every rounding midpoint and its neighbours,
  sub-normals, overflow and random values (bit for bit).
* :func:`value_scale_per_channel`, :func:`quantize_value_per_channel` -- pinned against
  torch's FP32 ``amax``/division/cast on the same inputs (bit for bit).
* :func:`attention_from_prepared` -- with the FP8 probability rounding and the FP16
  partial rounding switched off, pinned against an independent FP64 softmax on the
  dequantised operands (the frame shift, running maximum and weights then cancel
  exactly); closed form for a single key; the reference's SDPA envelope
  (``tests/attention/sage_attention_2pp/test_reference.py:12-35``).  Bit-level parity
  of the FP32 output with torch is *unpinned* (torch's exp and summation order), as for
  every non-torch implementation; outputs are compared by tolerance.
"""

from __future__ import annotations

import math

import numpy as np

from .piper_oracle import (
    DENOMINATOR_FLOOR,
    PV_BLOCK,
    SCALE_EPSILON,
    as_float32,
    quantize_query_key,
)

P_FP8_LN_MAX = np.float32(math.log(448.0))  # reference.py:17
V_FP8_MAX = np.float32(2.25)  # reference.py:18
FP8_MAX = 448.0
ACCUMULATE_MODES = ("reference", "fp32")


# --------------------------------------------------------------------------------------
# FP8 E4M3 (the "fn" variant: no infinities, 0x7F / 0xFF are NaN, max 448)
# --------------------------------------------------------------------------------------
def fp8_e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """Values of E4M3 codes (uint8) as float32: bias 7, 3 mantissa bits, sub-normals 2**-9 apart."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int32)
    sign = np.where(c & 0x80, -1.0, 1.0)
    exponent = (c >> 3) & 0xF
    mantissa = c & 0x7
    magnitude = np.where(
        exponent == 0,
        mantissa * 2.0**-9,
        (1.0 + mantissa / 8.0) * np.exp2(exponent.astype(np.float64) - 7.0),
    )
    value = sign * magnitude
    value = np.where((c & 0x7F) == 0x7F, np.nan, value)
    return value.astype(np.float32)


def fp8_e4m3_encode(x: np.ndarray) -> np.ndarray:
    """Round float32 to E4M3 codes, to nearest with ties to even (torch's ``float8_e4m3fn`` cast).

    Magnitudes that round above 448 (the largest code) and NaN/inf become NaN (0x7F with the
    sign), as the cast does.
    """
    x = np.asarray(x, dtype=np.float32)
    sign = (x.view(np.uint32) >> 31).astype(np.uint8) << 7
    a = np.abs(x).astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        # sub-normal range: multiples of 2**-9; code value k encodes k * 2**-9 for k <= 8
        sub = np.rint(a * 2.0**9)
        mant, exp = np.frexp(np.where(np.isfinite(a) & (a > 0), a, 1.0))  # a = mant * 2**exp, mant in [0.5, 1)
        e = exp - 1  # a = (2 mant) * 2**e, 2 mant in [1, 2)
        r = np.rint((2.0 * mant - 1.0) * 8.0)
        carry = r == 8.0
        r = np.where(carry, 0.0, r)
        e = np.where(carry, e + 1, e)
        normal = ((e + 7) * 8 + r).astype(np.int64)
    code = np.where(a < 2.0**-6, sub, normal)
    code = np.where(~np.isfinite(a) | (code > 0x7E), 0x7F, code).astype(np.uint8)
    return code | sign


def fp8_e4m3_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest E4M3 value, as float32."""
    return fp8_e4m3_decode(fp8_e4m3_encode(x))


# --------------------------------------------------------------------------------------
# V quantisation (reference.py:22-25)
# --------------------------------------------------------------------------------------
def value_scale_per_channel(v32: np.ndarray) -> np.ndarray:
    """``amax over the sequence of |v| / 2.25 + 1e-7`` in FP32, per (batch, head, channel)."""
    amax = np.abs(v32).max(axis=2).astype(np.float32)
    return (amax / V_FP8_MAX) + SCALE_EPSILON


def quantize_value_per_channel(v32: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """E4M3 codes of ``v / scale`` (IEEE FP32 division, then the E4M3 cast) and the scales."""
    scale = value_scale_per_channel(v32)
    quotient = (v32 / scale[:, :, None, :]).astype(np.float32)
    return fp8_e4m3_encode(quotient), scale


def prepare(q, k, v, granularity: str = "per_warp") -> dict:
    """Everything the reference derives before its key loop (reference.py:44-49)."""
    q32, k32, v32 = as_float32(q), as_float32(k), as_float32(v)
    prepared = quantize_query_key(q32, k32, granularity)
    v_codes, v_scale = quantize_value_per_channel(v32)
    prepared.update(value_code=v_codes, value_scale=v_scale)
    return prepared


# --------------------------------------------------------------------------------------
# streaming recurrence (reference.py:51-104)
# --------------------------------------------------------------------------------------
def attention_from_prepared(
    prepared: dict,
    scale: float,
    is_causal: bool,
    *,
    accumulate: str = "reference",
    query_offset: int = 0,
    quantize_probabilities: bool = True,
) -> np.ndarray:
    """The 64-key online-softmax loop and epilogue, in FP32. Returns the pre-cast output.

    ``accumulate="reference"``: each block's FP8 product is rounded to FP16 and scaled by
    the per-channel V scale before it is added (reference.py:95-99).  ``"fp32"``: the
    products accumulate in FP32 across blocks and the V scale is applied at the end.
    ``quantize_probabilities=False`` keeps FP32 probabilities (for pinning only).
    ``prepared`` may hold a contiguous subset of query rows starting at ``query_offset``.
    """
    if accumulate not in ACCUMULATE_MODES:
        raise ValueError(f"unknown accumulation mode: {accumulate}")
    q_code = prepared["query_code"]
    k_code = prepared["key_code"]
    v_val = fp8_e4m3_decode(prepared["value_code"]).astype(np.float64)
    q_scale = prepared["query_scale"].astype(np.float32)
    k_scale = prepared["key_scale"].astype(np.float32)
    v_scale = prepared["value_scale"].astype(np.float32)
    batch, heads, query_length, width = q_code.shape
    key_length = k_code.shape[2]
    scale32 = np.float32(scale)
    out = np.empty((batch, heads, query_length, width), dtype=np.float32)
    query_positions = np.arange(query_length) + query_offset
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        for b in range(batch):
            for h in range(heads):
                qf = q_code[b, h].astype(np.float32)
                accumulator = np.zeros((query_length, width), dtype=np.float32)
                denominator = np.zeros(query_length, dtype=np.float32)
                running_max = np.full(query_length, -np.inf, dtype=np.float32)
                for start in range(0, key_length, PV_BLOCK):
                    stop = min(start + PV_BLOCK, key_length)
                    integer_scores = qf @ k_code[b, h, start:stop].astype(np.float32).T
                    scores = integer_scores * q_scale[b, h, :, None] * k_scale[b, h, None, start:stop] * scale32
                    if is_causal:
                        future = np.arange(start, stop)[None, :] > query_positions[:, None]
                        scores = np.where(future, np.float32(-np.inf), scores)
                    block_max = scores.max(axis=-1) - P_FP8_LN_MAX
                    next_max = np.maximum(running_max, block_max)
                    old_weight = np.exp(running_max - next_max)
                    probabilities = np.nan_to_num(np.exp(scores - next_max[:, None]))
                    accumulator *= old_weight[:, None]
                    denominator = denominator * old_weight + probabilities.sum(axis=-1, dtype=np.float32)
                    p = fp8_e4m3_round(probabilities) if quantize_probabilities else probabilities
                    # FP8 x FP8 products are exact in FP64; the 64-term sums are rounded once to FP32
                    partial = (p.astype(np.float64) @ v_val[b, h, start:stop]).astype(np.float32)
                    if accumulate == "reference":
                        partial = partial.astype(np.float16).astype(np.float32)
                        accumulator += partial * v_scale[b, h][None, :]
                    else:
                        accumulator += partial
                    running_max = next_max
                if accumulate == "fp32":
                    accumulator = accumulator * v_scale[b, h][None, :]
                out[b, h] = accumulator / np.maximum(denominator, DENOMINATOR_FLOOR)[:, None]
    return out


def sage_attention_2pp_reference(
    q,
    k,
    v,
    scale: float | None = None,
    is_causal: bool = False,
    *,
    granularity: str = "per_warp",
    accumulate: str = "reference",
) -> np.ndarray:
    """Full quantised SageAttention2++ reference (reference.py:28-104); FP32 pre-cast output."""
    width = q.shape[-1]
    scale = width**-0.5 if scale is None else float(scale)
    prepared = prepare(q, k, v, granularity)
    return attention_from_prepared(prepared, scale, is_causal, accumulate=accumulate)

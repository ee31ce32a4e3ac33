"""CPU oracle for Piper Attention's forward pass (numpy restatement).

TEST INFRASTRUCTURE ONLY.  This module is the checker: it may be imported by
``tests/``, by ``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg of
``bench.py``, and by nothing else.  The product path (the ``piper_kernels``
package and its HIP library) never imports, calls or links it.

It restates, in numpy, the portable PyTorch reference of
``jumbledpoophj/piper-kernels`` 0.2.1:

* ``src/piper_kernels/attention/piper_attention/reference.py:22-118``
  (per-key V quantisation and the streaming UINT8-P / INT8-V recurrence);
* ``src/piper_kernels/attention/kernels/qk_quantization/int8/sage/reference.py:13-108``
  (K smoothing and INT8 Q/K quantisation, ``per_thread`` and ``per_warp``).

The sequence means of K and V (``reference.py:50``, ``sage/reference.py:89``:
FP32 ``torch.mean(dim=2)`` on CPU) are restated with torch's own summation
order (:func:`sequence_mean`): the FP32 cascade sum of torch's CPU reduction
kernel, then one FP32 division by S.  The HIP prep kernels compute the same
order, so K and V codes are bit-exact with the reference's portable path.

Parity status of each function (how it is pinned; see tests/test_oracle.py):

* ``sequence_mean`` -- pinned bit for bit against ``torch.mean(dim=2)`` on
  CPU (the reference's own call) over lengths, layouts and thread counts.
* ``quantize_per_group`` / ``quantize_*_per_thread`` / ``quantize_value_per_key``
  -- pinned by a pure-Python IEEE re-derivation on small inputs, the
  reference's own dequantisation bound (``tests/attention/test_qk_quantization.py:26-33``)
  and hand-written interleave tables for ``per_thread``.
* ``piper_attention_reference`` -- pinned by an independent FP64
  non-streaming restatement (``oracle/fp64_check.py``), closed forms for
  single-key and zero-query inputs, constant-V exactness, causal future
  independence and the reference's SDPA envelope.  Bit-level parity of the
  FP32 output with torch is *unpinned* (torch's exp/log/sum order), as it is
  for every non-torch implementation; outputs are compared by tolerance.
"""

from __future__ import annotations

import numpy as np

QUERY_BLOCK = 32  # sage/reference.py:6
KEY_BLOCK = 64  # sage/reference.py:7
PV_BLOCK = 64  # reference.py:16
MEAN_LEVELS = 4  # cascade levels of torch's CPU sum
INT8_RANGE = np.float32(127.0)  # sage/reference.py quantization_range / reference.py:18
P_UINT8_RANGE = np.float32(255.0)  # reference.py:17
SCALE_EPSILON = np.float32(1e-7)  # reference.py:19, sage/reference.py:8
DENOMINATOR_FLOOR = np.float32(1e-30)  # reference.py:116

GRANULARITIES = ("per_thread", "per_warp")


# --------------------------------------------------------------------------------------
# dtype plumbing
# --------------------------------------------------------------------------------------
def as_float32(x) -> np.ndarray:
    """Widen an fp16/bf16/fp32 array (numpy or torch) to a numpy float32 array, exactly."""
    if hasattr(x, "detach"):  # torch tensor: bf16 has no numpy dtype, widen in torch
        return x.detach().float().cpu().numpy()
    return np.asarray(x).astype(np.float32)


def round_to_bfloat16_bits(x32: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (round to nearest even), returned as uint16 bit patterns."""
    bits = np.ascontiguousarray(x32, dtype=np.float32).view(np.uint32)
    nan = np.isnan(x32)
    rounding_bias = ((bits >> 16) & 1) + np.uint32(0x7FFF)
    rounded = ((bits + rounding_bias) >> 16).astype(np.uint16)
    rounded[nan] = np.uint16(0x7FC0)
    return rounded


def bfloat16_bits_to_float32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def cast_output(out32: np.ndarray, dtype: str) -> np.ndarray:
    """Cast the FP32 result to the input dtype (reference.py:118), returned as float32 values.

    ``dtype`` is ``"float16"`` or ``"bfloat16"``.  Both casts round to nearest even.
    """
    if dtype == "float16":
        return out32.astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return bfloat16_bits_to_float32(round_to_bfloat16_bits(out32))
    raise ValueError(f"unsupported dtype {dtype}")


# --------------------------------------------------------------------------------------
# sequence mean (torch's CPU FP32 order)
# --------------------------------------------------------------------------------------
def cascade_block_rows(length: int) -> int:
    """Rows per first-level block of torch's cascade sum over ``length`` rows: 2**p with
    p = max(4, ceil(log2(length)) // 4) (16 for every length up to 2**19)."""
    ceil_log2 = (length - 1).bit_length() if length > 1 else 0
    return 1 << max(4, ceil_log2 // MEAN_LEVELS)


def cascade_sum(x32: np.ndarray) -> np.ndarray:
    """FP32 sum over axis 2 of ``[B, H, S, D]`` data in the order of torch's CPU reduction.

    Four accumulators start at +0.0.  Rows are added in order to level 0; after every block
    of L rows (L = :func:`cascade_block_rows`) level 0 is added to level 1 and cleared, and
    the carry continues upward -- level 1 into level 2 when the row count is a multiple of
    L**2, level 2 into level 3 when it is a multiple of L**3.  Trailing rows stay in level 0,
    and the result is ((level0 + level1) + level2) + level3.  Every addition rounds to FP32.
    """
    batch, heads, length, width = x32.shape
    step = cascade_block_rows(length)
    power = step.bit_length() - 1
    mask = step - 1
    acc = [np.zeros((batch, heads, width), dtype=np.float32) for _ in range(MEAN_LEVELS)]
    i = 0
    while i + step <= length:
        for _ in range(step):
            acc[0] = acc[0] + x32[:, :, i, :]
            i += 1
        for j in range(1, MEAN_LEVELS):
            acc[j] = acc[j] + acc[j - 1]
            acc[j - 1] = np.zeros_like(acc[j - 1])
            if i & (mask << (j * power)):
                break
    while i < length:
        acc[0] = acc[0] + x32[:, :, i, :]
        i += 1
    for j in range(1, MEAN_LEVELS):
        acc[0] = acc[0] + acc[j]
    return acc[0]


def sequence_mean(x32: np.ndarray) -> np.ndarray:
    """Mean over the sequence axis of ``[B, H, S, D]`` float32 data: :func:`cascade_sum`
    divided by S in FP32 (round to nearest even), which is what ``torch.mean(dim=2)`` returns
    on CPU for float32 input (``reference.py:50``, ``sage/reference.py:89``) when D is a
    multiple of 32 -- every head dim the operator accepts.  (torch's vectorised kernel takes
    columns in groups of 32 or 64 floats; a narrower remainder of columns is summed in another
    order, which this restatement does not model.)"""
    x32 = np.asarray(x32, dtype=np.float32)
    return (cascade_sum(x32) / np.float32(x32.shape[2])).astype(np.float32)


# --------------------------------------------------------------------------------------
# INT8 quantisers
# --------------------------------------------------------------------------------------
def _scale_from_amax(amax: np.ndarray, quantization_range: np.float32 = INT8_RANGE) -> np.ndarray:
    """``amax / range + 1e-7`` in FP32: IEEE division, then an FP32 add (sage/reference.py:68)."""
    amax = np.asarray(amax, dtype=np.float32)
    return (amax / np.float32(quantization_range)) + SCALE_EPSILON


def _codes(x32: np.ndarray, scale: np.ndarray, quantization_range=INT8_RANGE) -> np.ndarray:
    """``clamp(round_half_even(x / scale), -range, range)`` as int8 (sage/reference.py:70-75)."""
    quotient = x32 / scale
    r = np.float32(quantization_range)
    return np.clip(np.rint(quotient), -r, r).astype(np.int8)


def _pad_rows(x32: np.ndarray, multiple: int) -> tuple[np.ndarray, int]:
    """Zero-pad the sequence axis to a multiple (sage/reference.py:13-20)."""
    length = x32.shape[2]
    padded_length = -(-length // multiple) * multiple
    if padded_length == length:
        return x32, length
    padded = np.zeros(x32.shape[:2] + (padded_length, x32.shape[3]), dtype=np.float32)
    padded[:, :, :length] = x32
    return padded, length


def quantize_per_group(x32: np.ndarray, group: int, quantization_range=INT8_RANGE):
    """One scale per ``group`` consecutive rows (sage/reference.py:61-77).

    Returns ``(codes int8 [B,H,S,D], block_scale float32 [B,H,ceil(S/group)])``.
    """
    padded, length = _pad_rows(np.asarray(x32, dtype=np.float32), group)
    batch, heads, padded_length, width = padded.shape
    grouped = padded.reshape(batch, heads, padded_length // group, group * width)
    scale = _scale_from_amax(np.abs(grouped).max(axis=-1), quantization_range)
    codes = _codes(grouped, scale[..., None], quantization_range)
    return codes.reshape(batch, heads, padded_length, width)[:, :, :length], scale


def quantize_query_per_thread(q32: np.ndarray, quantization_range=INT8_RANGE):
    """Four interleaved query rows {t, t+8, t+16, t+24} share a scale (sage/reference.py:23-39).

    Returns ``(codes [B,H,S,D], per-row scale [B,H,S])``.
    """
    padded, length = _pad_rows(np.asarray(q32, dtype=np.float32), QUERY_BLOCK)
    batch, heads, padded_length, width = padded.shape
    # row = 32*block + 8*i + t  ->  axes (block, i, t, d); the scale group is (block, t)
    grouped = padded.reshape(batch, heads, padded_length // QUERY_BLOCK, 4, 8, width)
    group_scale = _scale_from_amax(np.abs(grouped).max(axis=(3, 5)), quantization_range)
    row_scale = np.broadcast_to(group_scale[:, :, :, None, :, None], grouped.shape)
    codes = _codes(grouped, row_scale, quantization_range).reshape(padded.shape)
    per_row = np.broadcast_to(group_scale[:, :, :, None, :], group_scale.shape[:3] + (4, 8))
    per_row = per_row.reshape(batch, heads, padded_length)
    return codes[:, :, :length], np.ascontiguousarray(per_row[:, :, :length])


def quantize_key_per_thread(k32: np.ndarray, quantization_range=INT8_RANGE):
    """Sixteen interleaved key rows {8a + 2t + c} share a scale (sage/reference.py:42-58).

    Returns ``(codes [B,H,S,D], per-row scale [B,H,S])``.
    """
    padded, length = _pad_rows(np.asarray(k32, dtype=np.float32), KEY_BLOCK)
    batch, heads, padded_length, width = padded.shape
    # row = 64*block + 8*a + 2*t + c -> axes (block, a, t, c, d); the scale group is (block, t)
    grouped = padded.reshape(batch, heads, padded_length // KEY_BLOCK, 8, 4, 2, width)
    group_scale = _scale_from_amax(np.abs(grouped).max(axis=(3, 5, 6)), quantization_range)
    row_scale = np.broadcast_to(group_scale[:, :, :, None, :, None, None], grouped.shape)
    codes = _codes(grouped, row_scale, quantization_range).reshape(padded.shape)
    per_row = np.broadcast_to(
        group_scale[:, :, :, None, :, None], group_scale.shape[:3] + (8, 4, 2)
    ).reshape(batch, heads, padded_length)
    return codes[:, :, :length], np.ascontiguousarray(per_row[:, :, :length])


def query_group_scales_per_thread(q32: np.ndarray, quantization_range=INT8_RANGE) -> np.ndarray:
    """The 8 group scales of every zero-padded 32-row Q block under ``per_thread``
    (group t = rows {t, t+8, t+16, t+24}): ``[B, H, Sq32/32, 8]``, the slots the HIP prep stores."""
    padded, _ = _pad_rows(np.asarray(q32, dtype=np.float32), QUERY_BLOCK)
    batch, heads, padded_length, width = padded.shape
    grouped = padded.reshape(batch, heads, padded_length // QUERY_BLOCK, 4, 8, width)
    return _scale_from_amax(np.abs(grouped).max(axis=(3, 5)), quantization_range)


def key_group_scales_per_thread(k_centered32: np.ndarray, quantization_range=INT8_RANGE) -> np.ndarray:
    """The 4 group scales of every zero-padded 64-row K block under ``per_thread``
    (group t = rows {8a + 2t + c}): ``[B, H, Sk64/64, 4]``."""
    padded, _ = _pad_rows(np.asarray(k_centered32, dtype=np.float32), KEY_BLOCK)
    batch, heads, padded_length, width = padded.shape
    grouped = padded.reshape(batch, heads, padded_length // KEY_BLOCK, 8, 4, 2, width)
    return _scale_from_amax(np.abs(grouped).max(axis=(3, 5, 6)), quantization_range)


def center_key(k32: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """``K - mean_S(K)`` in FP32 with the pinned mean (sage/reference.py:88-89)."""
    mean = sequence_mean(k32)
    return k32 - mean[:, :, None, :], mean


def quantize_query_key(q32: np.ndarray, k32: np.ndarray, granularity: str):
    """Centre K and quantise Q/K (sage/reference.py:80-108).

    Returns a dict with codes, per-row scales (as the reference returns them), for
    ``per_warp`` the per-block scales, and for both the scale slots the HIP prep stores
    (``query_slot_scale`` [B, H, Sq32/32, 8], ``key_slot_scale`` [B, H, Sk64/64, 4]: one per
    thread group, or the block scale repeated).
    """
    if granularity not in GRANULARITIES:
        raise ValueError(f"unknown Q/K quantization granularity: {granularity}")
    key_centered, key_mean = center_key(k32)
    result = {"key_mean": key_mean}
    if granularity == "per_warp":
        q_codes, q_block_scale = quantize_per_group(q32, QUERY_BLOCK)
        k_codes, k_block_scale = quantize_per_group(key_centered, KEY_BLOCK)
        result.update(
            query_code=q_codes,
            key_code=k_codes,
            query_block_scale=q_block_scale,
            key_block_scale=k_block_scale,
            query_scale=np.repeat(q_block_scale, QUERY_BLOCK, axis=2)[:, :, : q32.shape[2]],
            key_scale=np.repeat(k_block_scale, KEY_BLOCK, axis=2)[:, :, : k32.shape[2]],
            query_slot_scale=np.repeat(q_block_scale[..., None], 8, axis=3),
            key_slot_scale=np.repeat(k_block_scale[..., None], 4, axis=3),
        )
    else:
        q_codes, q_scale = quantize_query_per_thread(q32)
        k_codes, k_scale = quantize_key_per_thread(key_centered)
        result.update(
            query_code=q_codes,
            key_code=k_codes,
            query_scale=q_scale,
            key_scale=k_scale,
            query_slot_scale=query_group_scales_per_thread(q32),
            key_slot_scale=key_group_scales_per_thread(key_centered),
        )
    return result


def quantize_value_per_key(v_centered32: np.ndarray):
    """One signed-INT8 scale per V row (reference.py:22-32).

    Returns ``(codes int8 [B,H,S,D], scale float32 [B,H,S])``.
    """
    scale = _scale_from_amax(np.abs(v_centered32).max(axis=-1))
    return _codes(v_centered32, scale[..., None]), scale


def prepare(q, k, v, is_causal: bool, granularity: str = "per_warp") -> dict:
    """Everything the reference derives before its key loop (reference.py:45-59)."""
    q32, k32, v32 = as_float32(q), as_float32(k), as_float32(v)
    if is_causal:
        value_mean = np.zeros((v32.shape[0], v32.shape[1], v32.shape[3]), dtype=np.float32)
    else:
        value_mean = sequence_mean(v32)
    value_centered = v32 - value_mean[:, :, None, :]
    prepared = quantize_query_key(q32, k32, granularity)
    v_codes, v_scale = quantize_value_per_key(value_centered)
    prepared.update(value_code=v_codes, value_scale=v_scale, value_mean=value_mean)
    return prepared


# --------------------------------------------------------------------------------------
# streaming recurrence
# --------------------------------------------------------------------------------------
def attention_from_prepared(
    prepared: dict,
    scale: float,
    is_causal: bool,
    query_offset: int = 0,
    tie_window: float | None = None,
    flip_ties: bool = False,
):
    """The 64-key streaming loop and epilogue of reference.py:61-117, in FP32.

    Rows are independent, so ``prepared`` may hold a contiguous subset of the query rows
    (codes and per-row scales sliced alike); ``query_offset`` is the absolute position of
    its first row, used by the causal mask.

    Integer products are computed with FP32 matmuls, which are exact here: every partial
    sum is an integer of magnitude below 2**24 (|QK| <= 128*127**2, |PV| <= 64*255*127).
    Returns the FP32 output before the cast to the input dtype.

    With ``tie_window`` (a relative distance, e.g. 1e-5) it also returns, per query row, how
    far the output may move if every probability code whose unrounded value y = p * s_v * 255
    lies within ``tie_window * y`` of a rounding tie (a half integer) rounds the other way --
    what an implementation with other FP32 rounding (exp2/log2, operation order) can do.  A
    flip of code u_k by one moves output column d by v_code[k, d] * beta / 255 / den, carried
    by the same recurrence as the numerator, so the bound per row is that recurrence applied
    to sum_k max_d |v_code[k, d]| over the near-tie keys, divided by the final denominator:
    ``(out, flip_bound [B, H, Sq])``.  ``flip_ties=True`` (for testing that bound) rounds
    exactly those near-tie codes the other way.
    """
    q_code = prepared["query_code"]
    k_code = prepared["key_code"]
    v_code = prepared["value_code"]
    q_scale = prepared["query_scale"].astype(np.float32)
    k_scale = prepared["key_scale"].astype(np.float32)
    v_scale = prepared["value_scale"].astype(np.float32)
    v_mean = prepared["value_mean"]
    batch, heads, query_length, width = q_code.shape
    key_length = k_code.shape[2]
    scale32 = np.float32(scale)
    out = np.empty((batch, heads, query_length, width), dtype=np.float32)
    query_positions = np.arange(query_length) + query_offset
    flip_bound = np.zeros((batch, heads, query_length), dtype=np.float64) if tie_window is not None else None
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        for b in range(batch):
            for h in range(heads):
                qf = q_code[b, h].astype(np.float32)
                numerator = np.zeros((query_length, width), dtype=np.float32)
                denominator = np.zeros(query_length, dtype=np.float32)
                running_max = np.full(query_length, -np.inf, dtype=np.float32)
                flips = np.zeros(query_length, dtype=np.float64)  # the flip bound's numerator
                for start in range(0, key_length, PV_BLOCK):
                    stop = min(start + PV_BLOCK, key_length)
                    integer_scores = qf @ k_code[b, h, start:stop].astype(np.float32).T
                    scores = (
                        integer_scores
                        * q_scale[b, h, :, None]
                        * k_scale[b, h, None, start:stop]
                        * scale32
                    )
                    if is_causal:
                        future = np.arange(start, stop)[None, :] > query_positions[:, None]
                        scores = np.where(future, np.float32(-np.inf), scores)
                    block_v_scale = v_scale[b, h, start:stop]
                    shifted = scores + np.log(block_v_scale)[None, :]
                    block_max = shifted.max(axis=-1)
                    next_max = np.maximum(running_max, block_max)
                    old_weight = np.exp(running_max - next_max)
                    current_weight = np.exp(block_max - next_max)
                    probabilities = np.nan_to_num(np.exp(scores - block_max[:, None]))
                    numerator *= old_weight[:, None]
                    denominator = denominator * old_weight + probabilities.sum(axis=-1) * current_weight
                    unrounded = probabilities * block_v_scale[None, :] * P_UINT8_RANGE
                    p_codes = np.clip(np.rint(unrounded), np.float32(0.0), P_UINT8_RANGE)
                    if tie_window is not None:
                        y = unrounded.astype(np.float64)
                        tie = np.floor(y) + 0.5
                        near = (np.abs(y - tie) <= tie_window * np.maximum(y, 1.0)) & (tie < 255.0)
                        if flip_ties:  # round the near-tie codes the other way
                            other = np.where(p_codes > tie, np.floor(y), np.floor(y) + 1.0).astype(np.float32)
                            p_codes = np.where(near, other, p_codes)
                        vmax = np.abs(v_code[b, h, start:stop].astype(np.float64)).max(axis=-1)
                        weight64 = np.nan_to_num(current_weight.astype(np.float64))
                        flips = flips * np.nan_to_num(old_weight.astype(np.float64)) + (near @ vmax) * weight64 / 255.0
                    partial = p_codes @ v_code[b, h, start:stop].astype(np.float32)
                    numerator += partial * (current_weight / P_UINT8_RANGE)[:, None]
                    running_max = next_max
                result = numerator / np.maximum(denominator, DENOMINATOR_FLOOR)[:, None]
                result += v_mean[b, h][None, :]
                out[b, h] = result
                if flip_bound is not None:
                    flip_bound[b, h] = flips / np.maximum(denominator.astype(np.float64), float(DENOMINATOR_FLOOR))
    if flip_bound is not None:
        return out, flip_bound
    return out


def piper_attention_reference(
    q, k, v, scale: float | None = None, is_causal: bool = False, granularity: str = "per_thread"
) -> np.ndarray:
    """Full quantised reference (reference.py:35-118). Returns the FP32 pre-cast output.

    ``granularity`` defaults to ``per_thread`` like ``reference.py:42`` (the HIP operator's
    default too); ``per_warp`` is the per-block granularity of the reference's grouped path.
    """
    width = q.shape[-1]
    scale = width**-0.5 if scale is None else float(scale)
    prepared = prepare(q, k, v, is_causal, granularity)
    return attention_from_prepared(prepared, scale, is_causal)


# --------------------------------------------------------------------------------------
# full-precision quality reference
# --------------------------------------------------------------------------------------
def sdpa_float64(q, k, v, scale: float | None = None, is_causal: bool = False) -> np.ndarray:
    """Exact softmax attention in FP64 (the full-precision quality reference)."""
    q64 = as_float32(q).astype(np.float64)
    k64 = as_float32(k).astype(np.float64)
    v64 = as_float32(v).astype(np.float64)
    scale = q64.shape[-1] ** -0.5 if scale is None else float(scale)
    logits = np.einsum("bhqd,bhkd->bhqk", q64, k64) * scale
    if is_causal:
        sq, sk = logits.shape[-2:]
        logits = np.where(np.arange(sk)[None, :] > np.arange(sq)[:, None], -np.inf, logits)
    logits -= logits.max(axis=-1, keepdims=True)
    weights = np.exp(logits)
    weights /= weights.sum(axis=-1, keepdims=True)
    return np.einsum("bhqk,bhkd->bhqd", weights, v64)


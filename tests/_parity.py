"""Helpers shared by the GPU parity tests: run the HIP path, compare with the oracle."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"

# Gate of the attention output against the quantised oracle with matching (per-block)
# granularity, on the FP32 pre-cast output.  The kernel and the oracle evaluate the same
# formula with different FP32 rounding (exp2/log2 vs exp/log, operation order), so a P code
# can differ by one where p*vs*255 lies within rounding of a half integer; one such flip
# moves an output by |v_code| / (255 * den).  den grows with the key length, so short key
# sequences get a looser max-abs bound.  Mean error and cosine are gated tightly everywhere.
ATTENTION_MAX_ABS = 2e-3  # key length >= 1024
ATTENTION_MAX_ABS_SHORT = 1e-2  # key length < 1024
ATTENTION_MEAN_ABS = 1e-4
ATTENTION_COSINE = 0.9999


def max_abs_gate(key_length: int) -> float:
    return ATTENTION_MAX_ABS if key_length >= 1024 else ATTENTION_MAX_ABS_SHORT


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def load_golden(path: Path) -> dict:
    data = dict(np.load(path, allow_pickle=False))
    dtype = {"float16": torch.float16, "bfloat16": torch.bfloat16}[str(data["dtype"])]
    for name in ("query", "key", "value"):
        bits = torch.from_numpy(data[f"{name}_bits"].view(np.int16).copy())
        data[name] = bits.view(dtype)
    data["scale"] = float(data["scale"])
    data["is_causal"] = bool(data["is_causal"])
    return data


def gpu_prepare(q, k, v, scale, is_causal, device, plan=None, quantize_query=True, qk_granularity="per_warp"):
    from piper_kernels.attention.piper_attention.hip import _prepare_piper_attention

    with torch.no_grad():
        prepared = _prepare_piper_attention(
            q.to(device),
            k.to(device),
            v.to(device),
            scale,
            is_causal,
            plan=plan,
            quantize_query=quantize_query,
            qk_granularity=qk_granularity,
        )
    torch.cuda.synchronize(device)
    return prepared


def gpu_attention(prepared, dtype=torch.float32) -> torch.Tensor:
    from piper_kernels.attention.piper_attention.hip import _launch_piper_attention

    b, h, sq, _, d = prepared.shape
    out = torch.empty((b, h, sq, d), device=prepared.output.device, dtype=dtype)
    _launch_piper_attention(prepared, output=out)
    torch.cuda.synchronize(out.device)
    return out


def prepared_numpy(prepared) -> dict:
    b, h, sq, sk, d = prepared.shape
    vcode = prepared.value_code_transposed().cpu().numpy()  # [B,H,nkb,D,64]
    vcode = vcode.transpose(0, 1, 2, 4, 3).reshape(b, h, -1, d)
    return {
        "query_code_padded": prepared.query_code.cpu().numpy(),
        "query_slot_scale": None if prepared.query_scale is None else prepared.query_scale.cpu().numpy(),
        "key_code_padded": prepared.key_code().cpu().numpy(),
        "key_slot_scale": prepared.key_scale.cpu().numpy(),
        "key_tile_scale": prepared.key_tile_scale().cpu().numpy(),
        "value_code_padded": vcode,
        "value_scale_padded": prepared.value_scale.cpu().numpy(),
        "value_log2_scale": prepared.value_log2_scale().cpu().numpy(),
        "value_inv_multiplier": prepared.value_inv_multiplier().cpu().numpy(),
        "value_correction": prepared.value_correction().cpu().numpy(),
        "key_mean": prepared.key_mean.cpu().numpy(),
        "value_mean": prepared.value_mean.cpu().numpy(),
    }


def _bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and bool(np.array_equal(a.view(np.uint32), b.view(np.uint32)))


def _slots(expected: dict, name: str, slots: int) -> np.ndarray:
    """The scale slots the prep stores per block: the oracle's per-thread-group scales, or the
    per-block scale repeated (golden fixtures hold only the per-block ones)."""
    if f"{name}_slot_scale" in expected:
        return expected[f"{name}_slot_scale"]
    return np.repeat(np.asarray(expected[f"{name}_block_scale"])[..., None], slots, axis=-1)


def assert_prep_bit_exact(got: dict, expected: dict, shape, is_causal: bool) -> None:
    """Every code, scale and mean equal bit for bit; padding as documented in the header."""
    b, h, sq, sk, d = shape
    qc = got["query_code_padded"]
    assert np.array_equal(qc[:, :, :sq], expected["query_code"]), "query codes differ"
    assert not qc[:, :, sq:].any(), "query padding rows must be zero"
    assert _bits_equal(got["query_slot_scale"], _slots(expected, "query", 8)), "query scales differ"
    kc = got["key_code_padded"]
    assert np.array_equal(kc[:, :, :sk], expected["key_code"]), "key codes differ"
    assert not kc[:, :, sk:].any(), "key padding rows must be zero"
    assert _bits_equal(got["key_slot_scale"], _slots(expected, "key", 4)), "key scales differ"
    assert _bits_equal(got["key_tile_scale"], _slots(expected, "key", 4)), "tile copies of the key scales differ"
    assert _bits_equal(got["key_mean"], expected["key_mean"]), "key means differ"
    assert _bits_equal(got["value_mean"], expected["value_mean"]), "value means differ"
    if is_causal:
        assert not got["value_mean"].any()
    vc = got["value_code_padded"]
    mismatch = np.argwhere(vc[:, :, :sk] != expected["value_code"])
    assert mismatch.size == 0, f"value codes differ at {mismatch[:5].tolist()}"
    assert not vc[:, :, sk:].any(), "value padding keys must be zero"
    vs = got["value_scale_padded"]
    assert _bits_equal(vs[:, :, :sk], expected["value_scale"]), "value scales differ"
    # derived per-key arrays: exact IEEE reciprocal, log2 to library accuracy, padding masks
    inv_expected = np.float32(1.0) / (np.float32(255.0) * expected["value_scale"].astype(np.float32))
    assert _bits_equal(got["value_inv_multiplier"][:, :, :sk], inv_expected), "inverse multipliers differ"
    assert not got["value_inv_multiplier"][:, :, sk:].any()
    np.testing.assert_allclose(
        got["value_log2_scale"][:, :, :sk], np.log2(expected["value_scale"].astype(np.float64)), rtol=2e-7, atol=2e-7
    )
    assert np.all(np.isneginf(got["value_log2_scale"][:, :, sk:]))
    # affine correction = 128 * column sums of each 64-key tile
    codes = np.zeros((b, h, vc.shape[2], d), dtype=np.int64)
    codes[:, :, :sk] = expected["value_code"]
    colsum = codes.reshape(b, h, -1, 64, d).sum(axis=3)
    assert np.array_equal(got["value_correction"], 128 * colsum), "value correction differs"


def attention_metrics(actual: np.ndarray, expected: np.ndarray) -> dict:
    from piper_kernels.measure import measure_quality

    q = measure_quality(torch.from_numpy(np.asarray(actual, np.float32)), torch.from_numpy(np.asarray(expected, np.float32)))
    return q.as_dict()


def assert_attention_close(actual: np.ndarray, expected: np.ndarray, label: str = "",
                           max_abs: float | None = None, mean_abs: float = ATTENTION_MEAN_ABS,
                           cosine: float = ATTENTION_COSINE, key_length: int = 1) -> dict:
    if max_abs is None:
        max_abs = max_abs_gate(key_length)
    m = attention_metrics(actual, expected)
    log(f"[parity] {label} max_abs={m['max_absolute_error']:.3e} mean_abs={m['mean_absolute_error']:.3e} "
        f"cos={m['cosine_similarity']:.7f} sqnr={m['sqnr_db']:.2f}dB")
    assert np.all(np.isfinite(actual)), f"{label}: non-finite output"
    assert m["max_absolute_error"] <= max_abs, f"{label}: {m}"
    assert m["mean_absolute_error"] <= mean_abs, f"{label}: {m}"
    assert m["cosine_similarity"] >= cosine, f"{label}: {m}"
    return m

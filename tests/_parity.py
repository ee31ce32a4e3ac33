"""Helpers shared by the GPU parity tests: run the HIP path, compare with the oracle."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"

# Gate of the attention output against the quantised oracle with matching granularity, on the
# FP32 pre-cast output: max |err| <= 2e-3 in every row (the stated example tolerance), mean
# |err| <= 1e-4 and cosine >= 0.9999.  The kernel and the oracle evaluate the same formula with
# different FP32 rounding (exp2/log2 vs exp/log, operation order): their unrounded probability
# codes y = p * s_v * 255 agree to ~3e-6 relative, so a code whose y lies within that of a half
# integer may round the other way.  Such a flip moves the row by |v_code| * beta / (255 * den);
# the oracle bounds what all near-tie codes of a row can move it (TIE_WINDOW, a relative
# distance), and that bound is added to the row's 2e-3.
ATTENTION_MAX_ABS = 2e-3
ATTENTION_MEAN_ABS = 1e-4
ATTENTION_COSINE = 0.9999
TIE_WINDOW = 1e-5


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


def oracle_attention(prepared: dict, scale: float, is_causal: bool, query_offset: int = 0):
    """The oracle's FP32 output and its per-row tie-flip bound (see the gate above)."""
    from oracle import piper_oracle as oracle

    return oracle.attention_from_prepared(prepared, scale, is_causal, query_offset, tie_window=TIE_WINDOW)


def assert_attention_close(actual: np.ndarray, expected: np.ndarray, label: str = "",
                           flip_bound: np.ndarray | None = None, max_abs: float = ATTENTION_MAX_ABS,
                           mean_abs: float = ATTENTION_MEAN_ABS, cosine: float = ATTENTION_COSINE) -> dict:
    """Every row within max_abs (plus that row's tie-flip bound, [B, H, Sq], when given); mean
    error and cosine over the whole tensor."""
    m = attention_metrics(actual, expected)
    row_err = np.abs(np.asarray(actual, np.float64) - np.asarray(expected, np.float64)).max(axis=-1)
    allowed = max_abs + (0.0 if flip_bound is None else flip_bound)
    worst = np.unravel_index(int(np.argmax(row_err - allowed)), row_err.shape)
    flipped_rows = 0 if flip_bound is None else int((flip_bound > 0).sum())
    # rows whose error exceeds max_abs and pass only through their tie-flip allowance
    allowance_rows = int((row_err > max_abs).sum())
    log(f"[parity] {label} max_abs={m['max_absolute_error']:.3e} mean_abs={m['mean_absolute_error']:.3e} "
        f"cos={m['cosine_similarity']:.7f} sqnr={m['sqnr_db']:.2f}dB rows={row_err.size} "
        f"rows_with_near_ties={flipped_rows} rows_using_allowance={allowance_rows} "
        f"worst_row={tuple(int(i) for i in worst)} err={row_err[worst]:.3e} allowed={np.broadcast_to(allowed, row_err.shape)[worst]:.3e}")
    assert np.all(np.isfinite(actual)), f"{label}: non-finite output"
    assert (row_err <= allowed).all(), f"{label}: row {worst} error {row_err[worst]:.3e} beyond its gate; {m}"
    assert m["mean_absolute_error"] <= mean_abs, f"{label}: {m}"
    assert m["cosine_similarity"] >= cosine, f"{label}: {m}"
    return m

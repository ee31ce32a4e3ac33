"""The attention kernels' probability-code conversions on MI355X, through the kernels' own packers.

Piper Attention packs P codes with ``v_cvt_pk_u8_f32``; the reference rule it replaces is
``(p * v_scale * 255).round().clamp(0, 255)`` (reference.py:104-107), round half to even.  The
reference's own GPU test checks its NVIDIA packer on the edge values 0.49999997, 0.5, 254.5,
255.49998, 2^31 and FLT_MAX (tests/attention/piper_attention/test_triton.py:63-108); the same
values, every half-integer tie in [0, 256) and random values are checked here against numpy's
``clip(rint(x), 0, 255)``.  SageAttention2++ packs its P codes (values in [0, 448]) to FP8 E4M3
with ``v_cvt_pk_fp8_f32``; the reference casts with torch's ``float8_e4m3fn``
(sage_attention_2pp/reference.py:94), which the codes must equal bit for bit, ties included.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _parity import log
from piper_kernels.measure import probability_codes, scaled_probability_codes

pytestmark = pytest.mark.gpu

FLT_MAX = np.finfo(np.float32).max


def _u8_expected(values: np.ndarray) -> np.ndarray:
    return np.clip(np.rint(values), 0.0, 255.0).astype(np.uint8)


def test_u8_codes_on_the_reference_edge_values(gfx950_device) -> None:
    edges = np.array([0.49999997, 0.5, 254.5, 255.49998, 2.0**31, FLT_MAX], dtype=np.float32)
    log(f"[case] u8 codes of the reference's edge values {edges.tolist()}")
    got = probability_codes(edges, "u8", gfx950_device)
    assert got.tolist() == [0, 0, 254, 255, 255, 255]
    assert np.array_equal(got, _u8_expected(edges))


def test_u8_codes_round_half_to_even_and_saturate(gfx950_device) -> None:
    ties = np.arange(256, dtype=np.float32) + np.float32(0.5)  # every half-integer in [0.5, 255.5]
    near = np.concatenate([np.nextafter(ties, np.float32(0)), np.nextafter(ties, np.float32(512))])
    specials = np.array([0.0, -0.0, 1e-45, 1.0, 254.0, 255.0, 255.5, 256.0, 1e30, np.inf, -1.0, -0.5, -np.inf],
                        dtype=np.float32)
    rng = np.random.default_rng(7)
    uniform = rng.uniform(-8.0, 300.0, 20000).astype(np.float32)
    # the kernel's range: e = 255 * v_scale * p in [0, 255], as exp2 of a shifted score
    kernel_range = np.exp2(rng.uniform(-12.0, np.log2(255.0), 20000)).astype(np.float32)
    values = np.concatenate([ties, near, specials, uniform, kernel_range])
    log(f"[case] u8 codes of {values.size} values (ties, neighbours, specials, random)")
    got = probability_codes(values, "u8", gfx950_device)
    expected = _u8_expected(values)
    bad = np.flatnonzero(got != expected)
    assert bad.size == 0, f"{bad.size} codes differ, e.g. {values[bad[:8]].tolist()} -> {got[bad[:8]].tolist()}"
    assert got[:256].tolist() == [k + (k & 1) for k in range(256)][:255] + [255]  # k + 0.5 -> even neighbour


def test_scaled_u8_codes_round_the_exact_product_half_to_even(gfx950_device) -> None:
    """The kernel's subtraction-free path codes e = E * C with one FMA per code (E = exp2 of the
    shifted score, C = 2^(log2 255 - block max)): the code must be the exact product rounded half
    to even, for products in [0, 255.5)."""
    rng = np.random.default_rng(13)
    # the kernel's range: E = 2^x with x <= bm, C = 2^(log2 255 - bm), |bm| <= 96
    bm = rng.uniform(-96.0, 96.0, 4000).astype(np.float32)
    x = (bm[:, None] - rng.exponential(3.0, (4000, 4))).astype(np.float32)
    e_kernel = np.exp2(x.astype(np.float64)).astype(np.float32)
    c_kernel = np.exp2(np.float64(7.994353436858858) - bm.astype(np.float64)).astype(np.float32)
    # exact ties k + 1/2 and their float neighbours, split as (k + 1/2) 2^-j times 2^j
    k = np.arange(255, dtype=np.float64) + 0.5
    j = rng.integers(-60, 60, k.size).astype(np.float64)
    tie_e = (k * np.exp2(-j)).astype(np.float32)
    tie_c = np.exp2(j).astype(np.float32)
    tie_e = np.stack([tie_e, np.nextafter(tie_e, np.float32(0)), np.nextafter(tie_e, np.float32(np.inf)),
                      tie_e], axis=1)
    # empty rows: E = 0 (masked keys) with C = 0 or finite; the block maximum itself (E C ~ 255)
    special_e = np.array([[0.0, 0.0, 2.0**90, 2.0**-90]], dtype=np.float32)
    special_c = np.array([0.0], dtype=np.float32)
    top_e = np.exp2(bm[:8, None].astype(np.float64) * np.ones((8, 4))).astype(np.float32)
    values = np.concatenate([e_kernel, tie_e, np.zeros((1, 4), np.float32), special_e, top_e]).reshape(-1)
    mults = np.concatenate([c_kernel, tie_c, np.array([1.0], np.float32), special_c, c_kernel[:8]])
    product = values.astype(np.float64).reshape(-1, 4) * mults.astype(np.float64)[:, None]  # exact: 24 + 24 bits
    assert product.max() < 255.5
    log(f"[case] scaled u8 codes of {values.size} products (kernel range, ties, neighbours, empty rows)")
    got = scaled_probability_codes(values, mults, gfx950_device)
    expected = np.rint(product).reshape(-1).astype(np.uint8)
    bad = np.flatnonzero(got != expected)
    assert bad.size == 0, f"{bad.size} codes differ, e.g. {product.reshape(-1)[bad[:8]].tolist()} -> {got[bad[:8]].tolist()}"
    ties = got[4 * 4000: 4 * (4000 + 255)].reshape(255, 4)
    assert ties[:, 0].tolist() == [m + (m & 1) for m in range(255)]  # m + 1/2 -> the even neighbour
    assert got[4 * (4000 + 255 + 2): 4 * (4000 + 255 + 2) + 32].tolist() == [255] * 32  # the block maxima


def _e4m3_values() -> np.ndarray:
    """The non-negative finite FP8 E4M3 (fn) values, 0 .. 448, in increasing order."""
    codes = torch.arange(0, 0x7F, dtype=torch.uint8)  # 0x7F is NaN in the fn encoding
    return codes.view(torch.float8_e4m3fn).to(torch.float32).numpy()


def test_fp8_codes_match_torch_float8_e4m3fn(gfx950_device) -> None:
    grid = _e4m3_values()
    mids = (grid[:-1].astype(np.float64) + grid[1:]) / 2  # exact ties between neighbours (FP32-exact)
    mids = mids.astype(np.float32)
    assert np.array_equal(mids.astype(np.float64), (grid[:-1].astype(np.float64) + grid[1:]) / 2)
    near = np.concatenate([np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1024))])
    rng = np.random.default_rng(11)
    uniform = rng.uniform(0.0, 448.0, 20000).astype(np.float32)
    small = np.exp2(rng.uniform(-14.0, np.log2(448.0), 20000)).astype(np.float32)
    overshoot = np.array([448.0 * (1 + 2.0**-20), 448.0, 0.0, -0.0], dtype=np.float32)  # exp2 may land a hair above 448
    values = np.concatenate([grid, mids, near, uniform, small, overshoot])
    log(f"[case] fp8 codes of {values.size} values (grid, ties, neighbours, random, overshoot)")
    got = probability_codes(values, "fp8", gfx950_device)
    expected = torch.from_numpy(values).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    bad = np.flatnonzero(got != expected)
    assert bad.size == 0, f"{bad.size} codes differ, e.g. {values[bad[:8]].tolist()} -> {got[bad[:8]].tolist()}"
    assert np.array_equal(got[: grid.size], np.arange(0, 0x7F, dtype=np.uint8))  # every value maps to itself

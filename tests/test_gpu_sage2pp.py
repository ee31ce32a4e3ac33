"""SageAttention2++ on the GPU: the HIP path against the CPU oracle (oracle/sage2pp_oracle.py).

* Prep, bit for bit: K mean, INT8 K codes and per-block scales (and the copy of each scale in
  its tile record), per-channel V scales and FP8 E4M3 V codes; padding keys zero.
* Output, by tolerance, against the oracle in the kernel's own arithmetic (``accumulate="fp32"``:
  FP32 accumulation across blocks, V scale at the end) and in the reference's (FP16 partials).
  The remaining differences are exp2 versus exp, summation order and the rare FP8 probability
  that rounds the other way from within an ulp of a rounding midpoint (one such flip moves a
  probability by up to 1/16 of itself).  Gates: mean |err| <= 1e-4, cosine >= 0.99999 and
  max |err| <= 5e-3 against the FP32-accumulation oracle; against the reference mode, a mean no
  larger than the oracle's own distance between its two modes plus 1e-4 (that distance is the
  reference's FP16 rounding of each 64-key partial: up to 2e-4 on short sequences, where the
  partials are large); and the reference's own Triton-versus-reference gate (mean < 0.003,
  max < 0.12, tests/attention/sage_attention_2pp/test_triton.py:71-98) on its shapes.
* Invariants: every launch plan and a rerun give identical bits; strided views equal contiguous
  inputs; 16-bit outputs are the RNE rounding of the FP32 result; torch.compile(fullgraph=True).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _parity import GOLDEN, load_golden, log
from oracle import piper_oracle
from oracle import sage2pp_oracle as oracle
from piper_kernels.attention.piper_attention._plan import MI355XPlan

pytestmark = pytest.mark.gpu

MEAN_ABS = 1e-4
MAX_ABS = 5e-3
COSINE = 0.99999


def _prepare(q, k, v, scale, causal, device, plan=None, qk_granularity="per_warp"):
    from piper_kernels.attention.sage_attention_2pp.hip import _prepare_sage_attention_2pp

    with torch.no_grad():
        prepared = _prepare_sage_attention_2pp(
            q.to(device), k.to(device), v.to(device), scale, causal, plan=plan, qk_granularity=qk_granularity
        )
    torch.cuda.synchronize(device)
    return prepared


def _launch(prepared, dtype=torch.float32, accumulate="fp32") -> torch.Tensor:
    from piper_kernels.attention.sage_attention_2pp.hip import _launch_sage_attention_2pp

    b, h, sq, _, d = prepared.shape
    out = torch.empty((b, h, sq, d), device=prepared.output.device, dtype=dtype)
    _launch_sage_attention_2pp(prepared, output=out, accumulate=accumulate)
    torch.cuda.synchronize(out.device)
    return out


def _inputs(shape, dtype, seed):
    b, h, sq, sk, d = shape
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, h, sq, d, generator=g).to(dtype)
    k = (torch.randn(b, h, sk, d, generator=g) + 0.5 * torch.randn(b, h, 1, d, generator=g)).to(dtype)
    v = (torch.randn(b, h, sk, d, generator=g) * 1.5 + 0.5 * torch.randn(b, h, 1, d, generator=g)).to(dtype)
    return q, k, v


def _bits_equal(a, b) -> bool:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and bool(np.array_equal(a.view(np.uint32), b.view(np.uint32)))


def _cosine(a, b) -> float:
    a = a.astype(np.float64).ravel()
    b = b.astype(np.float64).ravel()
    return float(a @ b / np.sqrt((a @ a) * (b @ b)))


SHAPES = [
    # (B, H, Sq, Sk, D), dtype, causal
    ((1, 2, 65, 65, 64), torch.float16, False),
    ((2, 3, 35, 67, 128), torch.bfloat16, False),
    ((1, 1, 1, 1, 64), torch.float16, False),
    ((1, 2, 300, 1000, 128), torch.float16, False),
    ((1, 1, 193, 193, 128), torch.bfloat16, True),
    ((1, 2, 257, 257, 64), torch.float16, True),
]


def _id(case):
    shape, dtype, causal = case
    return "x".join(map(str, shape)) + f"-{str(dtype)[6:]}-c{int(causal)}"


@pytest.mark.parametrize("case", SHAPES, ids=_id)
def test_prep_bit_exact(gfx950_device, case) -> None:
    shape, dtype, causal = case
    log(f"[sage prep] {shape} {dtype} causal={causal}")
    b, h, sq, sk, d = shape
    q, k, v = _inputs(shape, dtype, seed=81)
    prepared = _prepare(q, k, v, d**-0.5, causal, gfx950_device)
    expected = oracle.prepare(q, k, v)
    assert _bits_equal(prepared.key_mean.cpu().numpy(), expected["key_mean"]), "key means differ"
    assert _bits_equal(prepared.key_scale.cpu().numpy(), expected["key_slot_scale"]), "key scales differ"
    tile_scale = prepared.kv_tiles[..., d : d + 16].contiguous().view(torch.float32).cpu().numpy()
    assert _bits_equal(tile_scale, expected["key_slot_scale"]), "tile copies of the key scales differ"
    kc = prepared.key_code().cpu().numpy()
    assert np.array_equal(kc[:, :, :sk], expected["key_code"]), "key codes differ"
    assert not kc[:, :, sk:].any(), "key padding rows must be zero"
    assert _bits_equal(prepared.value_scale.cpu().numpy(), expected["value_scale"]), "value scales differ"
    vc = prepared.value_code().cpu().numpy()
    mismatch = np.argwhere(vc[:, :, :sk] != expected["value_code"])
    assert mismatch.size == 0, f"value codes differ at {mismatch[:5].tolist()}"
    assert not vc[:, :, sk:].any(), "value padding keys must be zero"


@pytest.mark.parametrize("case", SHAPES, ids=_id)
def test_output_against_oracle(gfx950_device, case) -> None:
    shape, dtype, causal = case
    log(f"[sage attention] {shape} {dtype} causal={causal}")
    d = shape[-1]
    q, k, v = _inputs(shape, dtype, seed=82)
    prepared = _prepare(q, k, v, d**-0.5, causal, gfx950_device)
    actual = _launch(prepared).cpu().numpy()
    prep = oracle.prepare(q, k, v)
    fp32 = oracle.attention_from_prepared(prep, d**-0.5, causal, accumulate="fp32")
    reference = oracle.attention_from_prepared(prep, d**-0.5, causal)
    err = np.abs(actual - fp32)
    log(f"   vs fp32-accumulation oracle: mean {err.mean():.2e} max {err.max():.2e} cos {_cosine(actual, fp32):.7f}; "
        f"vs reference mode: mean {np.abs(actual - reference).mean():.2e} max {np.abs(actual - reference).max():.2e}")
    assert np.isfinite(actual).all()
    assert err.mean() <= MEAN_ABS and err.max() <= MAX_ABS and _cosine(actual, fp32) >= COSINE
    assert np.abs(actual - reference).mean() <= np.abs(fp32 - reference).mean() + MEAN_ABS
    # 16-bit outputs are the RNE rounding of the FP32 result
    out16 = _launch(prepared, dtype)
    assert torch.equal(out16.cpu(), torch.from_numpy(actual).to(dtype))


@pytest.mark.parametrize("case", SHAPES, ids=_id)
def test_fp16_partials_match_the_reference_mode(gfx950_device, case) -> None:
    """accumulate="reference" (PIPER_SAGE_FP16_PARTIALS) rounds each 64-key block's FP8 product to
    FP16 as the reference does (reference.py:95-98): against the oracle's reference mode it meets
    the gates the FP32 mode meets against the FP32 oracle, and it is nearer the reference mode than
    the FP32-accumulation oracle is wherever the two modes differ measurably."""
    shape, dtype, causal = case
    log(f"[sage fp16 partials] {shape} {dtype} causal={causal}")
    d = shape[-1]
    q, k, v = _inputs(shape, dtype, seed=86)
    prepared = _prepare(q, k, v, d**-0.5, causal, gfx950_device)
    actual = _launch(prepared, accumulate="reference").cpu().numpy()
    prep = oracle.prepare(q, k, v)
    reference = oracle.attention_from_prepared(prep, d**-0.5, causal)
    fp32 = oracle.attention_from_prepared(prep, d**-0.5, causal, accumulate="fp32")
    err = np.abs(actual - reference)
    modes = np.abs(fp32 - reference).mean()
    log(f"   vs reference mode: mean {err.mean():.2e} max {err.max():.2e} cos {_cosine(actual, reference):.7f}; "
        f"distance between the oracle's modes: mean {modes:.2e}")
    assert np.isfinite(actual).all()
    assert err.mean() <= MEAN_ABS and err.max() <= MAX_ABS and _cosine(actual, reference) >= COSINE
    if modes > 1e-5:
        assert err.mean() < modes
    out16 = _launch(prepared, dtype, accumulate="reference")
    assert torch.equal(out16.cpu(), torch.from_numpy(actual).to(dtype))


@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_reference_gate(gfx950_device, dtype, head_dim, is_causal) -> None:
    """tests/attention/sage_attention_2pp/test_triton.py:71-98 with this oracle as the reference."""
    from piper_kernels import sage_attention_2pp

    torch.manual_seed(43)
    query = torch.randn(1, 2, 193, head_dim, dtype=dtype)
    key = torch.randn_like(query)
    value = torch.randn_like(query)
    with torch.no_grad():
        actual = sage_attention_2pp(query.to(gfx950_device), key.to(gfx950_device), value.to(gfx950_device),
                                    is_causal=is_causal)
    expected = piper_oracle.cast_output(
        oracle.sage_attention_2pp_reference(query, key, value, head_dim**-0.5, is_causal, granularity="per_thread"),
        str(dtype)[6:],
    )
    error = np.abs(actual.float().cpu().numpy() - expected)
    assert actual.shape == query.shape and actual.dtype is dtype
    assert torch.isfinite(actual).all()
    assert error.mean() < 0.003 and error.max() < 0.12


def test_plans_and_reruns_are_bitwise_identical(gfx950_device) -> None:
    q, k, v = _inputs((1, 2, 700, 700, 128), torch.bfloat16, seed=83)
    outs = []
    for plan in [p for p in MI355XPlan.all_plans() if not p.work_queue] + [MI355XPlan()]:  # no work queue here
        prepared = _prepare(q, k, v, 128**-0.5, True, gfx950_device, plan=plan)
        outs.append(_launch(prepared).cpu())
    assert all(torch.equal(outs[0], o) for o in outs[1:])


def test_strided_inputs_match_contiguous(gfx950_device) -> None:
    from piper_kernels import sage_attention_2pp

    torch.manual_seed(84)
    base = torch.randn(1, 100, 3, 4, 128, dtype=torch.float16, device=gfx950_device)
    q, k, v = (base[:, :, i].transpose(1, 2) for i in range(3))
    with torch.no_grad():
        strided = sage_attention_2pp(q, k, v)
        dense = sage_attention_2pp(q.contiguous(), k.contiguous(), v.contiguous())
    assert torch.equal(strided, dense)


def test_torch_compile_fullgraph(gfx950_device) -> None:
    from piper_kernels import sage_attention_2pp

    torch.manual_seed(85)
    qs = torch.randn(3, 2, 128, 64, device=gfx950_device, dtype=torch.float16)
    ks, vs = torch.randn_like(qs), torch.randn_like(qs)
    q, k, v = (t.permute(1, 0, 2, 3) for t in (qs, ks, vs))

    def consumer(q, k, v):
        return -sage_attention_2pp(q, k, v)

    with torch.no_grad():
        expected = consumer(q, k, v)
        actual = torch.compile(consumer, fullgraph=True)(q, k, v)
    assert torch.equal(actual, expected)


def test_quality_against_fp64_sdpa(gfx950_device) -> None:
    """The reference's own envelope against exact attention (test_reference.py:12-35) at a
    longer length, and the same distance to SDPA as the quantised reference."""
    from piper_kernels import sage_attention_2pp

    torch.manual_seed(86)
    q = torch.randn(1, 2, 1024, 128, dtype=torch.float16)
    k, v = torch.randn_like(q), torch.randn_like(q)
    with torch.no_grad():
        actual = sage_attention_2pp(q.to(gfx950_device), k.to(gfx950_device), v.to(gfx950_device)).float().cpu().numpy()
    sdpa = piper_oracle.sdpa_float64(q, k, v)
    reference = oracle.sage_attention_2pp_reference(q, k, v, granularity="per_thread")  # the operator's default
    err, ref_err = np.abs(actual - sdpa), np.abs(reference - sdpa)
    log(f"[sage sdpa] max {err.max():.3e} (reference {ref_err.max():.3e}) cos {_cosine(actual, sdpa):.6f}")
    assert err.mean() < 0.01 and err.max() < 0.2
    assert err.max() <= ref_err.max() + 2e-3
    assert _cosine(actual, sdpa) >= _cosine(reference, sdpa) - 1e-5


GOLDEN_FIXTURES = sorted((GOLDEN / "sage2pp").glob("*.npz"))


@pytest.mark.parametrize(
    "plan", [MI355XPlan(waves=8), MI355XPlan(waves=4), MI355XPlan(waves=4, three_per_cu=True)], ids=["w8", "w4", "w3"]
)
@pytest.mark.parametrize("fixture", GOLDEN_FIXTURES, ids=[p.stem for p in GOLDEN_FIXTURES])
def test_golden_fixture(gfx950_device, fixture, plan) -> None:
    """Prep bit for bit and the output within the gates of the committed oracle fixtures."""
    g = load_golden(fixture)
    log(f"[sage golden] {fixture.stem} plan={plan.plan_id}")
    q, k, v = g["query"], g["key"], g["value"]
    sk, d = k.shape[2], k.shape[3]
    prepared = _prepare(q, k, v, g["scale"], g["is_causal"], gfx950_device, plan=plan)
    assert _bits_equal(prepared.key_mean.cpu().numpy(), g["key_mean"])
    assert _bits_equal(prepared.key_scale.cpu().numpy(), np.repeat(g["key_block_scale"][..., None], 4, axis=-1))
    assert _bits_equal(prepared.value_scale.cpu().numpy(), g["value_scale"])
    assert np.array_equal(prepared.key_code().cpu().numpy()[:, :, :sk], g["key_code"])
    assert np.array_equal(prepared.value_code().cpu().numpy()[:, :, :sk], g["value_code"])
    actual = _launch(prepared).cpu().numpy()
    err = np.abs(actual - g["output_fp32_accumulation"])
    assert err.mean() <= MEAN_ABS and err.max() <= MAX_ABS
    modes = np.abs(g["output_fp32_accumulation"] - g["output_reference"]).mean()
    assert np.abs(actual - g["output_reference"]).mean() <= modes + MEAN_ABS


@pytest.mark.parametrize("case", SHAPES, ids=_id)
def test_per_thread_granularity(gfx950_device, case) -> None:
    """The default of the reference's portable path (reference.py:35, "per_thread"): K codes and
    the four K group scales bit for bit, and the output (query quantised per thread group in
    the prologue) against the oracle's per_thread restatement in the kernel's arithmetic."""
    shape, dtype, causal = case
    log(f"[sage per_thread] {shape} {dtype} causal={causal}")
    b, h, sq, sk, d = shape
    g = torch.Generator().manual_seed(83)
    # every thread group its own magnitude: query row r x (1 + (r % 8) / 8), key row r x (1 + ((r % 8) // 2) / 4)
    q = (torch.randn(b, h, sq, d, generator=g) * (1 + (torch.arange(sq) % 8).reshape(1, 1, sq, 1) / 8)).to(dtype)
    k = (torch.randn(b, h, sk, d, generator=g) * (1 + (torch.arange(sk) % 8 // 2).reshape(1, 1, sk, 1) / 4)
         + 0.5 * torch.randn(b, h, 1, d, generator=g)).to(dtype)
    v = (torch.randn(b, h, sk, d, generator=g) + 2.0 * torch.randn(b, h, 1, d, generator=g)).to(dtype)
    prepared = _prepare(q, k, v, d**-0.5, causal, gfx950_device, qk_granularity="per_thread")
    prep = oracle.prepare(q, k, v, "per_thread")
    assert _bits_equal(prepared.key_scale.cpu().numpy(), prep["key_slot_scale"]), "key scales differ"
    assert np.array_equal(prepared.key_code().cpu().numpy()[:, :, :sk], prep["key_code"]), "key codes differ"
    actual = _launch(prepared).cpu().numpy()
    fp32 = oracle.attention_from_prepared(prep, d**-0.5, causal, accumulate="fp32")
    err = np.abs(actual - fp32)
    log(f"   vs fp32-accumulation oracle: mean {err.mean():.2e} max {err.max():.2e}")
    assert np.isfinite(actual).all()
    assert err.mean() <= MEAN_ABS and err.max() <= MAX_ABS and _cosine(actual, fp32) >= COSINE

"""Measurement semantics restated from the reference's benchmark harness.

* ``attention_operations`` -- the operation count of
  ``benchmarks/benchmark_attention.py:184-193``: 4*B*H*pairs*D, pairs = Sq*Skv, or the
  causal triangle Sq*(Sq+1)/2.
* ``measure_quality`` -- the metrics defined in ``benchmarks/lib/quality.py:88-252`` (mean/max
  absolute error, relative L1/L2 error, SQNR in dB and cosine similarity over the finite pairs,
  non-finite values counted separately), evaluated in float64 on the host.

``measure_mfma_peak`` has no counterpart in the reference (whose benchmarks quote published
peaks only): it times the library's back-to-back MFMA probe to give the sustained dense
matrix-core rate of the GPU at hand, which the attention kernels are priced against next to
the published 5.0 P/s.  ``measure_mfma_valu_sharing`` (no counterpart either) times the
same probe's MFMA-only, FMA-only and interleaved kinds at the attention kernels' occupancy, to
show how much MFMA execution and VALU issue overlap on a SIMD.
"""

from __future__ import annotations

import math
from dataclasses import asdict, dataclass

import torch

INT8_DENSE_PEAK_TOPS = 5033.2  # MI355X: 256 CU x 2.4 GHz x 8192 int8 ops/clk/CU (dense)
HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E


def attention_operations(
    batch: int, heads: int, query_length: int, key_length: int, head_dim: int, is_causal: bool
) -> int:
    pairs = query_length * key_length
    if is_causal:
        pairs = query_length * (query_length + 1) // 2
    return 4 * batch * heads * pairs * head_dim


def effective_tops(operations: int, milliseconds: float) -> float:
    return operations / (milliseconds * 1e-3) / 1e12


@dataclass(frozen=True)
class QualityMetrics:
    """Error of an output against a reference (field names as in the benchmark records)."""

    mean_absolute_error: float
    max_absolute_error: float
    relative_l1_error: float
    relative_l2_error: float
    sqnr_db: float
    cosine_similarity: float
    actual_nonfinite_count: int
    reference_nonfinite_count: int
    nonfinite_mismatch_count: int

    def as_dict(self) -> dict:
        return asdict(self)


def _as_float64_vector(tensor: torch.Tensor) -> torch.Tensor:
    if tensor.dtype in (torch.int64, torch.uint64):
        # float64 holds integers exactly only up to 2^53
        raise ValueError("64-bit integer tensors cannot be compared exactly in float64")
    return tensor.detach().reshape(-1).to(device="cpu", dtype=torch.float64)


def _sqnr_db(signal_energy: float, noise_energy: float) -> float:
    if noise_energy == 0.0:
        return math.inf if signal_energy > 0.0 else math.nan
    return 10.0 * math.log10(signal_energy / noise_energy) if signal_energy > 0.0 else -math.inf


def _cosine(x: torch.Tensor, y: torch.Tensor) -> float:
    xx, yy = float(x.square().sum()), float(y.square().sum())
    if xx == 0.0 or yy == 0.0:
        return 1.0 if xx == yy else 0.0  # two zero vectors agree; a zero and a non-zero do not
    return max(-1.0, min(1.0, float(torch.dot(x, y)) / math.sqrt(xx * yy)))


def measure_quality(actual: torch.Tensor, reference: torch.Tensor) -> QualityMetrics:
    """Error of ``actual`` against ``reference`` (same shape, any floating or small integer dtype).

    The metric definitions are those of the reference's benchmark harness
    (``benchmarks/lib/quality.py:88-252``); everything is evaluated in float64 on the host:

    * over the positions where both tensors are finite, with e = actual - reference: mean and
      max of |e|, relative L1 error sum|e| / sum|reference|, relative L2 error
      ||e||_2 / ||reference||_2, SQNR = 10 log10(sum reference^2 / sum e^2) dB and the cosine
      of the angle between the two vectors;
    * counts of non-finite values in each tensor, and of positions where at least one is
      non-finite and they disagree (NaN against NaN, or the same infinity, agrees).

    With no finite pair every error metric is NaN.
    """
    if actual.shape != reference.shape:
        raise ValueError(f"shape mismatch: actual {tuple(actual.shape)}, reference {tuple(reference.shape)}")
    x = _as_float64_vector(actual)
    y = _as_float64_vector(reference)
    x_ok, y_ok = torch.isfinite(x), torch.isfinite(y)
    same = (x == y) | (torch.isnan(x) & torch.isnan(y))
    counts = (
        int((~x_ok).sum()),
        int((~y_ok).sum()),
        int(((~x_ok | ~y_ok) & ~same).sum()),
    )
    pairs = x_ok & y_ok
    if not bool(pairs.any()):
        return QualityMetrics(*([math.nan] * 6), *counts)
    x, y = x[pairs], y[pairs]
    error = x - y
    magnitude = error.abs()
    tiny = torch.finfo(torch.float64).tiny
    signal_energy = float(y.square().sum())
    noise_energy = float(error.square().sum())
    return QualityMetrics(
        mean_absolute_error=float(magnitude.mean()),
        max_absolute_error=float(magnitude.max()),
        relative_l1_error=float(magnitude.sum()) / max(float(y.abs().sum()), tiny),
        relative_l2_error=math.sqrt(noise_energy) / max(math.sqrt(signal_energy), tiny),
        sqnr_db=_sqnr_db(signal_energy, noise_energy),
        cosine_similarity=_cosine(x, y),
        actual_nonfinite_count=counts[0],
        reference_nonfinite_count=counts[1],
        nonfinite_mismatch_count=counts[2],
    )


def prep_algorithmic_bytes(
    batch: int,
    heads: int,
    query_length: int,
    key_length: int,
    head_dim: int,
    is_causal: bool,
    quantize_query: bool = True,
) -> int:
    """Minimum HBM bytes of the prep stage: fp16/bf16 reads of Q, K, V, int8 code writes,
    FP32 scales (Q per 32 rows, K per 64 rows, V per key) and the K/V means.  Without the
    query (``quantize_query=False``: the attention kernel quantises it) only K and V count."""
    eq = batch * heads * query_length * head_dim if quantize_query else 0
    ekv = batch * heads * key_length * head_dim
    q_scales = -(-query_length // 32) if quantize_query else 0
    scales = 4 * batch * heads * (q_scales + -(-key_length // 64) + key_length)
    means = (4 if is_causal else 8) * batch * heads * head_dim
    return 2 * (eq + 2 * ekv) + (eq + 2 * ekv) + scales + means


def sage_prep_algorithmic_bytes(batch: int, heads: int, key_length: int, head_dim: int) -> int:
    """Minimum HBM bytes of the SageAttention2++ prep: fp16/bf16 reads of K and V, INT8 K and
    FP8 V code writes, FP32 K scales (per 64 rows), K means and per-channel V scales."""
    ekv = batch * heads * key_length * head_dim
    scales = 4 * batch * heads * (-(-key_length // 64) + 2 * head_dim)
    return 2 * 2 * ekv + 2 * ekv + scales


def mfma_probe_expected(kind: int, iterations: int) -> int:
    """The 32-bit word every probe thread stores: the sum of its 64 accumulators, each
    ``iterations * K`` with all-ones operands (K = 32 INT8, 64 FP8); FP8 as FP32 bits."""
    from ._hip import library as native

    import struct

    if kind == native.MFMA_PROBE_I8:
        return (iterations * 2048) % (1 << 32)
    if kind in (native.MFMA_PROBE_VALU, native.MFMA_PROBE_VALU_LDS):  # 16 chains of 4 * iterations + 1.0
        return struct.unpack("<I", struct.pack("<f", float(iterations * 64)))[0]
    if kind == native.MFMA_PROBE_I8_VALU:
        return (iterations * 2048 + iterations * 64) % (1 << 32)
    if kind == native.MFMA_PROBE_MAX3:  # 16 chains that stay at 1.0
        return struct.unpack("<I", struct.pack("<f", 16.0))[0]
    if kind == native.MFMA_PROBE_EXP:
        raise ValueError("the exp probe converges to an irrational value: check it with exp_probe_ok")
    if kind in (native.MFMA_PROBE_P_CODES_U8, native.MFMA_PROBE_P_CODES_FP8):
        raise ValueError("the conversion kinds store codes of their input values: use probability_codes")
    return struct.unpack("<I", struct.pack("<f", float(iterations * 4096)))[0]


EXP_PROBE_FIXED_POINT = 0.6411857445049859  # the root of x = 2^-x


def exp_probe_ok(words) -> bool:
    """Every thread of the exp probe converged to the same 16-chain sum, 16 * the root of
    x = 2^-x to within v_exp_f32's accuracy."""
    import numpy as np

    values = np.asarray(words, dtype=np.uint32).view(np.float32)
    return bool((values == values[0]).all() and abs(float(values[0]) - 16 * EXP_PROBE_FIXED_POINT) < 1e-4)


def probability_codes(values, codes: str, device: torch.device):
    """The attention kernels' probability codes of FP32 ``values``, computed on the GPU by the
    kernels' own packers (the probe's conversion kinds): ``codes="u8"`` gives Piper Attention's
    UINT8 codes u (the packer's bytes u - 128, shifted back), ``codes="fp8"``
    SageAttention2++'s FP8 E4M3 bit patterns.  Returns a uint8 array of the same length."""
    import numpy as np

    from ._hip import library as native

    kinds = {"u8": native.MFMA_PROBE_P_CODES_U8, "fp8": native.MFMA_PROBE_P_CODES_FP8}
    if codes not in kinds:
        raise ValueError(f"codes must be 'u8' or 'fp8', got {codes!r}")
    flat = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    per_group = native.MFMA_PROBE_THREADS  # values read by one workgroup; it packs them into 128 words
    workgroups = max(1, -(-flat.size // per_group))
    host = np.zeros(workgroups * per_group, dtype=np.float32)
    host[: flat.size] = flat
    sink = torch.from_numpy(host.view(np.int32)).to(device)
    stream = torch.cuda.current_stream(device)
    with torch.cuda.device(device):
        native.load_library().mfma_probe(kinds[codes], workgroups, 1, sink.data_ptr(), stream.cuda_stream)
        stream.synchronize()
    words = sink.cpu().numpy().view(np.uint32).reshape(workgroups, 4, per_group // 4)
    if not (words == words[:, :1]).all():  # thread t and t + 128k pack the same four values
        raise RuntimeError("probability-code probe: threads packing the same values disagree")
    packed = np.ascontiguousarray(words[:, 0]).view(np.uint8).reshape(-1)  # little-endian: value 4i + j in byte j of word i
    if codes == "u8":
        packed = packed ^ np.uint8(0x80)
    return packed[: flat.size]


def _time_probe(lib, kind: int, workgroups: int, iterations: int, launches: int, device: torch.device) -> float:
    """Median milliseconds of ``launches`` probe launches (after two warm-ups); the result
    words are checked against their exact value."""
    from ._hip import library as native

    sink = torch.zeros(workgroups * native.MFMA_PROBE_THREADS, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device)
    with torch.cuda.device(device):
        for _ in range(2):
            lib.mfma_probe(kind, workgroups, iterations, sink.data_ptr(), stream.cuda_stream)
        times = []
        for _ in range(launches):
            begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            begin.record(stream)
            lib.mfma_probe(kind, workgroups, iterations, sink.data_ptr(), stream.cuda_stream)
            end.record(stream)
            end.synchronize()
            times.append(begin.elapsed_time(end))
    words = sink.cpu().numpy().view("uint32")
    if kind == native.MFMA_PROBE_EXP:
        if not exp_probe_ok(words):
            raise RuntimeError("MFMA probe kind exp returned wrong results")
    else:
        expected = mfma_probe_expected(kind, iterations)
        if not (words == expected).all():
            raise RuntimeError(f"MFMA probe kind {kind} returned wrong results ({int((words != expected).sum())} threads)")
    return sorted(times)[len(times) // 2]


def measure_mfma_peak(kind: int, device: torch.device, *, iterations: int = 4096, launches: int = 5) -> dict:
    """Sustained dense MFMA rate (tera-ops/s) of the library's probe on ``device``.

    Four workgroups of 8 waves per compute unit, four independent accumulator chains per wave;
    the median of ``launches`` timed launches (HIP events on the launch stream) after two
    warm-up launches.  Every thread's result word is checked against its exact value, so a
    time cannot come from elided work.  ``iterations <= 4096`` keeps the FP8 check exact.
    """
    from ._hip import library as native

    lib = native.load_library()
    workgroups = 4 * torch.cuda.get_device_properties(device).multi_processor_count
    ms = _time_probe(lib, kind, workgroups, iterations, launches, device)
    ops = workgroups * (native.MFMA_PROBE_THREADS // 64) * 4 * iterations * native.MFMA_PROBE_OPS[kind]
    return {
        "instruction": "v_mfma_i32_32x32x32_i8" if kind == native.MFMA_PROBE_I8 else "v_mfma_f32_32x32x64_f8f6f4",
        "tops": round(ops / (ms * 1e-3) / 1e12, 1),
        "ms_per_launch": round(ms, 4),
        "workgroups": workgroups,
        "iterations": iterations,
    }


def measure_mfma_valu_sharing(device: torch.device, *, iterations: int = 2048, launches: int = 5) -> dict:
    """How INT8 MFMA execution and FP32 VALU issue share a SIMD at the attention kernels'
    occupancy (one 8-wave workgroup per compute unit: two waves per SIMD).

    Times the probe's MFMA-only, FMA-only and interleaved kinds (4 MFMAs and 64 FMAs per
    wave-round).  ``overlap`` = (t_mfma + t_valu - t_both) / min(t_mfma, t_valu): 1 when the
    units run concurrently, 0 when MFMA execution and VALU issue serialise.  The cycle figures
    convert per-SIMD time at the 2.4 GHz peak clock: per MFMA, per FMA (two waves issuing), and
    the VALU cycles one interleaved MFMA costs (its share of t_both - t_valu); and, from the
    max3 and exp kinds, the per-SIMD cycles of a v_max3_f32 and a v_exp_f32 issued by two waves;
    and, from the LDS kind, the VALU cycles one interleaved wave-wide ds_read_b128 costs.
    """
    from ._hip import library as native

    if iterations > 1 << 18:
        raise ValueError("iterations must be <= 2^18 for the exact FMA check")
    lib = native.load_library()
    workgroups = torch.cuda.get_device_properties(device).multi_processor_count
    kinds = (native.MFMA_PROBE_I8, native.MFMA_PROBE_VALU, native.MFMA_PROBE_I8_VALU, native.MFMA_PROBE_MAX3,
             native.MFMA_PROBE_EXP, native.MFMA_PROBE_VALU_LDS)
    t = {k: _time_probe(lib, k, workgroups, iterations, launches, device) for k in kinds}
    t_m, t_v, t_b = t[native.MFMA_PROBE_I8], t[native.MFMA_PROBE_VALU], t[native.MFMA_PROBE_I8_VALU]
    cycles = 2.4e9 * 1e-3  # cycles per millisecond at the peak clock
    waves_per_simd = native.MFMA_PROBE_THREADS // 64 // 4
    mfmas = waves_per_simd * 4 * iterations  # per SIMD
    fmas = waves_per_simd * 64 * iterations
    return {
        "workgroups": workgroups,
        "iterations": iterations,
        "mfma_ms": round(t_m, 4),
        "valu_ms": round(t_v, 4),
        "both_ms": round(t_b, 4),
        "overlap": round((t_m + t_v - t_b) / min(t_m, t_v), 3),
        "cycles_per_mfma": round(t_m * cycles / mfmas, 1),
        "cycles_per_fma": round(t_v * cycles / fmas, 2),
        "cycles_per_max3": round(t[native.MFMA_PROBE_MAX3] * cycles / fmas, 2),
        "cycles_per_exp": round(t[native.MFMA_PROBE_EXP] * cycles / fmas, 2),
        "valu_cycles_per_lds_read": round((t[native.MFMA_PROBE_VALU_LDS] - t_v) * cycles / (fmas / 8), 1),
        "valu_cycles_per_interleaved_mfma": round((t_b - t_v) * cycles / mfmas, 1),
    }

"""Measurement semantics restated from the reference's benchmark harness.

* ``attention_operations`` -- the operation count of
  ``benchmarks/benchmark_attention.py:184-193``: 4*B*H*pairs*D, pairs = Sq*Skv, or the
  causal triangle Sq*(Sq+1)/2.
* ``measure_quality`` -- the metrics defined in ``benchmarks/lib/quality.py:88-252`` (mean/max
  absolute error, relative L1/L2 error, SQNR in dB and cosine similarity over the finite pairs,
  non-finite values counted separately), evaluated in float64 on the host.

``measure_mfma_peak`` has no counterpart in the reference (whose benchmarks quote published
peaks only): it times the measurement library's back-to-back MFMA probe to give the sustained
dense matrix-core rate of the GPU at hand, which the attention kernels are priced against next
to the published 5.0 P/s.  ``measure_issue_sharing`` (no counterpart either) runs the issue
probe's per-wave roles side by side on shared SIMDs, to show how VALU issue scales with waves
per SIMD and how much MFMA execution, VALU issue and LDS reads of different waves overlap --
the issue bound of the attention kernels.
"""

from __future__ import annotations

import ctypes
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
    if kind == native.MFMA_PROBE_F8:
        return struct.unpack("<I", struct.pack("<f", float(iterations * 4096)))[0]
    raise ValueError("the conversion kinds store codes of their input values: use probability_codes")


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
        native.load_probe_library().mfma_probe(kinds[codes], workgroups, 1, sink.data_ptr(), stream.cuda_stream)
        stream.synchronize()
    words = sink.cpu().numpy().view(np.uint32).reshape(workgroups, 4, per_group // 4)
    if not (words == words[:, :1]).all():  # thread t and t + 128k pack the same four values
        raise RuntimeError("probability-code probe: threads packing the same values disagree")
    packed = np.ascontiguousarray(words[:, 0]).view(np.uint8).reshape(-1)  # little-endian: value 4i + j in byte j of word i
    if codes == "u8":
        packed = packed ^ np.uint8(0x80)
    return packed[: flat.size]


def scaled_probability_codes(values, multipliers, device: torch.device):
    """Piper Attention's UINT8 codes of the products ``values[4i + j] * multipliers[i]``,
    computed on the GPU by the kernels' scaled packer (the subtraction-free exp2 path: one FMA
    per code with the block's multiplier).  ``values`` holds 4N FP32 values, ``multipliers`` N;
    returns the 4N codes u (the packer's bytes u - 128, shifted back) as uint8."""
    import numpy as np

    from ._hip import library as native

    flat = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    mult = np.ascontiguousarray(multipliers, dtype=np.float32).reshape(-1)
    if flat.size != 4 * mult.size:
        raise ValueError(f"need four values per multiplier, got {flat.size} values and {mult.size} multipliers")
    groups = 64  # groups of four values per workgroup
    workgroups = max(1, -(-mult.size // groups))
    host = np.zeros((workgroups, native.MFMA_PROBE_THREADS), dtype=np.float32)
    padded = np.zeros(workgroups * groups * 4, dtype=np.float32)
    padded[: flat.size] = flat
    host[:, :256] = padded.reshape(workgroups, 256)
    pm = np.zeros(workgroups * groups, dtype=np.float32)
    pm[: mult.size] = mult
    host[:, 256::4] = pm.reshape(workgroups, groups)
    sink = torch.from_numpy(host.reshape(-1).view(np.int32)).to(device)
    stream = torch.cuda.current_stream(device)
    with torch.cuda.device(device):
        native.load_probe_library().mfma_probe(native.MFMA_PROBE_P_CODES_U8_SCALED, workgroups, 1, sink.data_ptr(),
                                               stream.cuda_stream)
        stream.synchronize()
    words = sink.cpu().numpy().view(np.uint32).reshape(workgroups, native.MFMA_PROBE_THREADS // groups, groups)
    if not (words == words[:, :1]).all():  # thread t and t + 64k pack the same four values
        raise RuntimeError("scaled probability-code probe: threads packing the same values disagree")
    packed = np.ascontiguousarray(words[:, 0]).view(np.uint8).reshape(-1) ^ np.uint8(0x80)
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
    expected = mfma_probe_expected(kind, iterations)
    if not (words == expected).all():
        raise RuntimeError(f"MFMA probe kind {kind} returned wrong results ({int((words != expected).sum())} threads)")
    return sorted(times)[len(times) // 2]


def measure_mfma_peak(kind: int, device: torch.device, *, iterations: int = 4096, launches: int = 5) -> dict:
    """Sustained dense MFMA rate (tera-ops/s) of the measurement library's probe on ``device``.

    Four workgroups of 8 waves per compute unit, four independent accumulator chains per wave;
    the median of ``launches`` timed launches (HIP events on the launch stream) after two
    warm-up launches.  Every thread's result word is checked against its exact value, so a
    time cannot come from elided work.  ``iterations <= 4096`` keeps the FP8 check exact.
    """
    from ._hip import library as native

    lib = native.load_probe_library()
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


# instructions per round of each issue-probe role (include/piper_probe.h)
ISSUE_ROUND = {
    "mfma": {"mfma": 2},
    "fma": {"valu": 32},
    "exp": {"valu": 32},
    "cvt": {"valu": 32},
    "mix": {"mfma": 2, "valu": 44},
    "valu_mix": {"valu": 44},
    "lds": {"lds": 16},
    "mfma_fma": {"mfma": 2, "valu": 32},
    "mix_vgpr": {"mfma": 2, "valu": 44},
    "cluster": {"mfma": 8, "valu": 176},
    "add_lit": {"valu": 32},
    "add_sgpr": {"valu": 32},
    "fma_split": {"valu": 32},
    "fma_same": {"valu": 32},
    "fmac_same": {"valu": 32},
    "max3": {"valu": 32},
    "perm": {"valu": 32},
}


def run_issue_probe(device: torch.device, roles: list[str], *, cycle_budget: int = 400_000) -> dict:
    """One launch of the issue probe (after a warm-up launch) with ``roles[s]`` for slot s of every
    SIMD (len(roles) waves per SIMD, one workgroup per CU).  Per role: ticks per round, the
    s_memtime ticks one SIMD takes for one round of that role (a wave's ticks divided by the rounds
    all of that role's waves on its SIMD completed, the median over SIMDs), and the fewest and most
    rounds a single wave completed (an uneven split shows starvation).  Every SIMD must hold
    exactly len(roles) waves of the workgroup."""
    import numpy as np

    from ._hip import library as native

    if not 1 <= len(roles) <= native.ISSUE_MAX_WAVES_PER_SIMD:
        raise ValueError("one to four roles")
    codes = [native.ISSUE_ROLES.index(r) for r in roles]
    lib = native.load_probe_library()
    workgroups = torch.cuda.get_device_properties(device).multi_processor_count
    count = workgroups * native.ISSUE_RECORDS_PER_WORKGROUP
    records = torch.full((count * ctypes.sizeof(native.PiperIssueRecord),), 255, dtype=torch.uint8, device=device)
    args = native.PiperIssueProbeArgs(waves_per_simd=len(roles), workgroups=workgroups, cycle_budget=cycle_budget,
                                      records=records.data_ptr())
    for i, c in enumerate(codes):
        args.roles[i] = c
    stream = torch.cuda.current_stream(device)
    with torch.cuda.device(device):
        for _ in range(2):
            lib.issue_probe(args, stream.cuda_stream)
        stream.synchronize()
    raw = records.cpu().numpy().view(
        np.dtype([("hw_id", "<u4"), ("xcc_id", "<u4"), ("role", "<u4"), ("slot", "<u4"), ("cycles", "<u8"),
                  ("rounds", "<u4"), ("check", "<u4")])
    ).reshape(workgroups, native.ISSUE_RECORDS_PER_WORKGROUP)[:, : 4 * len(roles)].reshape(-1)
    if (raw["hw_id"] == 0xFFFFFFFF).any():
        raise RuntimeError("issue probe: a wave wrote no record")
    hw = raw["hw_id"].astype(np.int64)
    simd_key = ((raw["xcc_id"].astype(np.int64) & 15) << 20) | (((hw >> 12) & 15) << 12) | (((hw >> 8) & 15) << 4) | ((hw >> 4) & 3)
    per_role: dict[str, list[float]] = {r: [] for r in set(roles) if r != "idle"}
    spread: dict[str, list[int]] = {r: [] for r in per_role}
    keys, inverse, counts = np.unique(simd_key, return_inverse=True, return_counts=True)
    if (counts != len(roles)).any():
        raise RuntimeError(f"issue probe: SIMDs hold {sorted(set(counts.tolist()))} waves, expected {len(roles)}")
    for simd in range(len(keys)):
        waves = raw[inverse == simd]
        for role in per_role:
            mine = waves[waves["role"] == native.ISSUE_ROLES.index(role)]
            if len(mine) == 0 or mine["rounds"].sum() == 0:
                continue
            per_role[role].append(float(mine["cycles"].max()) / float(mine["rounds"].sum()))
            spread[role].extend(mine["rounds"].tolist())
    return {
        "roles": roles,
        "simds": int(len(keys)),
        **{
            role: {"ticks_per_round": round(float(np.median(v)), 2), "wave_rounds": [min(spread[role]), max(spread[role])]}
            for role, v in per_role.items()
        },
    }


def measure_issue_sharing(device: torch.device, *, cycle_budget: int = 400_000) -> dict:
    """How the SIMD shares issue between waves (the issue probe; s_memtime ticks, which count at
    the shader clock):

    * ``valu_ticks_per_instruction``: FP32 FMA, v_cvt_pk_u8_f32 and v_exp_f32 throughput of a SIMD
      with 1-4 waves issuing only that class (a single wave issues at most one instruction per
      ~6 ticks; the pipes take 2, 4 and 8 ticks per wave-wide instruction);
    * ``mfma_ticks``: one v_mfma_i32_32x32x32_i8 of a wave issuing only MFMAs;
    * ``cross_wave``: an MFMA-only wave beside one or three FMA-only waves: both rates next to
      their rates alone;
    * ``in_wave``: MFMA and FMA interleaved in one wave (AGPR accumulators), one and two waves
      per SIMD;
    * ``attention_mix``: three waves per SIMD of the attention loop's mix (per MFMA 16 FMA,
      4 cvt_pk_u8, 2 exp) with and without its MFMAs; ``mfma_cost_ticks`` is what one MFMA adds
      to the SIMD's time, against its ``mfma_ticks`` duration (0: fully overlapped, equal:
      serialised);
    * ``lds``: wave-wide ds_read_b128 throughput of a CU (four waves per SIMD reading) in bytes
      per tick, and the attention mix with an LDS-reading wave beside it;
    * ``mfma_placement``: the attention mix's MFMA cost with VGPR instead of AGPR accumulators,
      and with the MFMAs bunched eight at a time (per round 8 MFMAs then 176 VALU instructions)
      instead of spread one per 22 VALU instructions;
    * ``operand``: v_add_f32 ticks per instruction with a 32-bit literal and with an SGPR
      operand, three waves per SIMD (an FP32 VALU instruction reading an SGPR issues at half
      the rate);
    * ``vgpr_banks``: v_fma_f32 with its sources in three different VGPR banks (register number
      mod 4) and with its first two sources in one bank, and v_fmac_f32 with its accumulator in
      the bank of its first source, three waves per SIMD (a bank conflict costs the FP32 pipe
      extra cycles);
    * ``valu_class``: v_max3_f32 and v_perm_b32 (the attention loop's row maximum and code
      packing), sources in different banks, three waves per SIMD, beside ``vgpr_banks``'
      conflict-free FMA.
    """

    def run(*roles: str) -> dict:
        return run_issue_probe(device, list(roles), cycle_budget=cycle_budget)

    def per_instr(result: dict, role: str, kind: str) -> float:
        return round(result[role]["ticks_per_round"] / ISSUE_ROUND[role][kind], 2)

    valu = {}
    for role in ("fma", "cvt", "exp"):
        valu[role] = {str(n): per_instr(run(*([role] * n)), role, "valu") for n in (1, 2, 3, 4)}
    mfma_alone = run("mfma")
    fma_alone = run("fma")
    mfma_ticks = per_instr(mfma_alone, "mfma", "mfma")
    pair = run("mfma", "fma")
    quad = run("mfma", "fma", "fma", "fma")
    fma3 = run("fma", "fma", "fma")
    in1 = run("mfma_fma")
    in2 = run("mfma_fma", "mfma_fma")
    fma2 = run("fma", "fma")
    mix3 = run("mix", "mix", "mix")
    vmix3 = run("valu_mix", "valu_mix", "valu_mix")
    lds4 = run("lds", "lds", "lds", "lds")
    vmix_lds = run("valu_mix", "valu_mix", "valu_mix", "lds")
    mixv3 = run("mix_vgpr", "mix_vgpr", "mix_vgpr")
    cluster3 = run("cluster", "cluster", "cluster")
    lit3 = run("add_lit", "add_lit", "add_lit")
    sgpr3 = run("add_sgpr", "add_sgpr", "add_sgpr")
    banked = {role: per_instr(run(role, role, role), role, "valu") for role in ("fma_split", "fma_same", "fmac_same", "max3", "perm")}
    vmix_round = vmix3["valu_mix"]["ticks_per_round"]
    return {
        "ticks": "s_memtime",
        "cycle_budget": cycle_budget,
        "valu_ticks_per_instruction": valu,
        "mfma_ticks": mfma_ticks,
        "cross_wave": {
            "mfma_plus_fma": {"mfma_ticks": per_instr(pair, "mfma", "mfma"), "fma_ticks": per_instr(pair, "fma", "valu"),
                              "fma_alone_ticks": per_instr(fma_alone, "fma", "valu")},
            "mfma_plus_3_fma": {"mfma_ticks": per_instr(quad, "mfma", "mfma"),
                                "fma_ticks": per_instr(quad, "fma", "valu"),
                                "fma_alone_ticks": per_instr(fma3, "fma", "valu")},
        },
        "in_wave": {
            "one_wave_round_ticks": in1["mfma_fma"]["ticks_per_round"],
            "one_wave_fma_alone_ticks": fma_alone["fma"]["ticks_per_round"],
            "two_waves_round_ticks": in2["mfma_fma"]["ticks_per_round"],
            "two_waves_fma_alone_ticks": fma2["fma"]["ticks_per_round"],
            "mfma_only_round_ticks": mfma_alone["mfma"]["ticks_per_round"],
        },
        "attention_mix": {
            "mix_round_ticks": mix3["mix"]["ticks_per_round"],
            "valu_mix_round_ticks": vmix3["valu_mix"]["ticks_per_round"],
            "mfma_cost_ticks": round((mix3["mix"]["ticks_per_round"] - vmix3["valu_mix"]["ticks_per_round"]) / 2, 2),
            "mfma_ticks": mfma_ticks,
        },
        "lds": {
            "bytes_per_tick_per_cu": round(4 * 16 * 1024 / lds4["lds"]["ticks_per_round"], 1),
            "valu_mix_round_ticks_beside_lds_wave": vmix_lds["valu_mix"]["ticks_per_round"],
        },
        "mfma_placement": {
            "agpr_spread_mfma_cost_ticks": round((mix3["mix"]["ticks_per_round"] - vmix_round) / 2, 2),
            "vgpr_spread_mfma_cost_ticks": round((mixv3["mix_vgpr"]["ticks_per_round"] - vmix_round) / 2, 2),
            "agpr_bunched_mfma_cost_ticks": round((cluster3["cluster"]["ticks_per_round"] - 4 * vmix_round) / 8, 2),
        },
        "operand": {
            "add_literal_ticks": per_instr(lit3, "add_lit", "valu"),
            "add_sgpr_ticks": per_instr(sgpr3, "add_sgpr", "valu"),
        },
        "vgpr_banks": {
            "fma_distinct_banks_ticks": banked["fma_split"],
            "fma_src0_src1_same_bank_ticks": banked["fma_same"],
            "fmac_accumulator_src0_same_bank_ticks": banked["fmac_same"],
        },
        "valu_class": {
            "fma_ticks": banked["fma_split"],
            "max3_ticks": banked["max3"],
            "perm_ticks": banked["perm"],
        },
    }


class ClockProbe:
    """The engine clock a workload runs at, read on the GPU itself: the measurement library's
    clock probe (``piper_clock_probe``) runs one sleeping wave per XCC on a stream of its own,
    beside the workload on the caller's stream, and reads the variable-frequency shader clock
    counter against the constant-rate wall clock counter over its life.  Reads only; the clock
    is never set.  Usage: queue some of the workload, ``start()``, keep queueing until
    ``done()``, then ``summary()``."""

    def __init__(self, device: torch.device, duration_ms: float = 300.0, workgroups: int = 8) -> None:
        from ._hip.library import load_probe_library

        self.device = device
        self.duration_us = int(duration_ms * 1000)
        self.workgroups = workgroups
        self._lib = load_probe_library()
        self.records = torch.zeros(4 * workgroups, dtype=torch.int64, device=device)
        self.stream = torch.cuda.Stream(device)  # default priority
        self.wall_khz = 0

    def start(self) -> None:
        self.wall_khz = self._lib.clock_probe(self.workgroups, self.duration_us, self.records.data_ptr(),
                                              self.stream.cuda_stream)

    def done(self) -> bool:
        return self.stream.query()

    def summary(self) -> dict:
        """Per-wave engine clocks in MHz (one wave per XCC when workgroups = XCCs): median,
        range, and the wall time the waves spanned."""
        import statistics

        self.stream.synchronize()
        r = self.records.cpu().tolist()
        mhz, wall_ms = [], []
        for g in range(self.workgroups):
            wall0, clock0, wall1, clock1 = r[4 * g: 4 * g + 4]
            if wall1 > wall0:
                mhz.append((clock1 - clock0) / (wall1 - wall0) * self.wall_khz / 1000.0)
                wall_ms.append((wall1 - wall0) / self.wall_khz)
        if not mhz:
            return {"engine_clock_mhz_median": None}
        return {
            "engine_clock_mhz_median": round(statistics.median(mhz), 1),
            "engine_clock_mhz_min_max": [round(min(mhz), 1), round(max(mhz), 1)],
            "probe_waves": len(mhz),
            "probe_wall_ms": round(statistics.median(wall_ms), 1),
            "wall_clock_khz": self.wall_khz,
        }



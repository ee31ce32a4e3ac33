"""The measurement library's probes on MI355X.

* The dense MFMA probe: every thread's accumulator sum is exact (so the timed MFMAs really ran)
  and the measured rate is below the published dense peak at the 2.4 GHz maximum clock (a
  counting check) and above a tenth of it (the probe saturates).
* The issue probe: every wave writes its record, every SIMD holds the requested waves, and the
  rates are physical: one MFMA takes at least the 32 cycles its 65536 operations need at
  2048 per cycle, and more FMA waves per SIMD never make the SIMD's FMA throughput worse.
"""

from __future__ import annotations

import pytest

from _parity import log
from piper_kernels._hip import library as native
from piper_kernels.measure import INT8_DENSE_PEAK_TOPS, measure_issue_sharing, measure_mfma_peak, run_issue_probe

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", [native.MFMA_PROBE_I8, native.MFMA_PROBE_F8], ids=["int8", "fp8"])
def test_mfma_probe_rate(gfx950_device, kind) -> None:
    log(f"[probe] kind {kind}")
    result = measure_mfma_peak(kind, gfx950_device, iterations=1024, launches=3)  # raises on a wrong word
    log(f"   {result}")
    # both instructions have the same dense peak on MI355X: 5.0 P/s at 2.4 GHz
    assert 0.1 * INT8_DENSE_PEAK_TOPS < result["tops"] <= 1.001 * INT8_DENSE_PEAK_TOPS


def test_issue_probe_records_and_rates(gfx950_device) -> None:
    log("[probe] issue probe: mfma alone, fma at 1 and 4 waves, mixed roles")
    mfma = run_issue_probe(gfx950_device, ["mfma"], cycle_budget=100_000)
    fma1 = run_issue_probe(gfx950_device, ["fma"], cycle_budget=100_000)
    fma4 = run_issue_probe(gfx950_device, ["fma"] * 4, cycle_budget=100_000)
    mixed = run_issue_probe(gfx950_device, ["mfma", "fma", "lds", "idle"], cycle_budget=100_000)
    log(f"   {mfma}\n   {fma1}\n   {fma4}\n   {mixed}")
    assert mfma["simds"] == fma4["simds"] == 4 * 256
    assert mfma["mfma"]["ticks_per_round"] / 2 >= 31.0  # 2 MFMAs per round, >= 32 cycles each
    assert fma4["fma"]["ticks_per_round"] <= fma1["fma"]["ticks_per_round"] * 1.05
    assert {"mfma", "fma", "lds"} <= set(mixed) and "idle" not in mixed


def test_issue_sharing_summary(gfx950_device) -> None:
    """The bench's issue-sharing record is complete and consistent."""
    result = measure_issue_sharing(gfx950_device, cycle_budget=100_000)
    log(f"[probe] {result}")
    valu = result["valu_ticks_per_instruction"]
    assert set(valu) == {"fma", "cvt", "exp"} and all(set(v) == {"1", "2", "3", "4"} for v in valu.values())
    assert valu["exp"]["4"] >= valu["fma"]["4"]  # exp is a quarter-rate instruction
    assert result["mfma_ticks"] >= 31.0 and result["lds"]["bytes_per_tick_per_cu"] > 0
    placement = result["mfma_placement"]
    assert all(0.0 < v < 2 * result["mfma_ticks"] for v in placement.values()), placement
    assert result["operand"]["add_literal_ticks"] > 0 and result["operand"]["add_sgpr_ticks"] > 0
    banks, classes = result["vgpr_banks"], result["valu_class"]
    assert all(v > 0 for v in (*banks.values(), *classes.values())), (banks, classes)
    # a bank conflict never makes an FMA faster
    assert banks["fma_src0_src1_same_bank_ticks"] >= 0.95 * banks["fma_distinct_banks_ticks"], banks


def test_clock_probe_reads_a_physical_engine_clock(gfx950_device) -> None:
    """The clock probe's waves span at least the requested wall time, and the shader clock they read
    lies between the idle floor and the 2.4 GHz maximum; beside a busy MFMA probe the clock is up."""
    import time

    import torch

    from piper_kernels.measure import ClockProbe

    log("[probe] clock probe, 30 ms, 8 waves, alone and beside the MFMA probe")
    probe = ClockProbe(gfx950_device, duration_ms=30.0, workgroups=8)
    probe.start()
    alone = probe.summary()
    log(f"   alone {alone}")
    assert alone["probe_waves"] == 8 and alone["wall_clock_khz"] > 0
    assert alone["probe_wall_ms"] >= 30.0
    assert 20.0 < alone["engine_clock_mhz_min_max"][0] <= alone["engine_clock_mhz_min_max"][1] <= 2400.0 * 1.01
    busy = ClockProbe(gfx950_device, duration_ms=30.0, workgroups=8)
    lib = native.load_probe_library()
    sink = torch.empty(1024 * native.MFMA_PROBE_THREADS, dtype=torch.int32, device=gfx950_device)
    stream = torch.cuda.current_stream(gfx950_device)
    lib.mfma_probe(native.MFMA_PROBE_I8, 1024, 4096, sink.data_ptr(), stream.cuda_stream)
    busy.start()
    guard = time.perf_counter()
    while not busy.done() and time.perf_counter() - guard < 5.0:
        lib.mfma_probe(native.MFMA_PROBE_I8, 1024, 4096, sink.data_ptr(), stream.cuda_stream)
        stream.synchronize()
    beside = busy.summary()
    log(f"   beside MFMA work {beside}")
    assert beside["probe_waves"] == 8 and 500.0 < beside["engine_clock_mhz_median"] <= 2400.0 * 1.01

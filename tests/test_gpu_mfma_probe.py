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

"""The roofline-calibration probe on MI355X: every thread's accumulator sum is exact (so the
timed MFMAs really ran) and the measured rate is below the published dense peak at the
2.4 GHz maximum clock (a counting check) and above a tenth of it (the probe saturates); the
MFMA/VALU sharing kinds return exact words and time between overlap and serialisation."""

from __future__ import annotations

import pytest

from _parity import log
from piper_kernels._hip import library as native
from piper_kernels.measure import INT8_DENSE_PEAK_TOPS, measure_mfma_peak, measure_mfma_valu_sharing

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", [native.MFMA_PROBE_I8, native.MFMA_PROBE_F8], ids=["int8", "fp8"])
def test_mfma_probe_rate(gfx950_device, kind) -> None:
    log(f"[probe] kind {kind}")
    result = measure_mfma_peak(kind, gfx950_device, iterations=1024, launches=3)  # raises on a wrong word
    log(f"   {result}")
    # both instructions have the same dense peak on MI355X: 5.0 P/s at 2.4 GHz
    assert 0.1 * INT8_DENSE_PEAK_TOPS < result["tops"] <= 1.001 * INT8_DENSE_PEAK_TOPS


def test_mfma_valu_sharing_probe(gfx950_device) -> None:
    """The MFMA-only, FMA-only and interleaved probe kinds return exact words (checked inside),
    and the interleaved time lies between full overlap and full serialisation (with a margin
    for clock noise)."""
    log("[probe] MFMA/VALU sharing")
    result = measure_mfma_valu_sharing(gfx950_device, iterations=1024, launches=3)
    log(f"   {result}")
    t_m, t_v, t_b = result["mfma_ms"], result["valu_ms"], result["both_ms"]
    assert 0.95 * max(t_m, t_v) <= t_b <= 1.05 * (t_m + t_v)
    assert -0.1 <= result["overlap"] <= 1.1

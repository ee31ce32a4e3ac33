"""The kernels' quantisation codes equal clip(rint(x / s), -127, 127) with IEEE division.

``csrc/quant.h`` computes the code of x in two steps, once per element:

* the quotient RN(x / s) as fma(fma(-s, q0, x), y, q0) with y = RN(1/s) and q0 = RN(x * y)
  (``Divisor``), instead of an IEEE division per element;
* the rounded code as the low byte of the bits of RN(quotient + 1.5 * 2^23) (``code_word``),
  instead of rint, a clamp and a conversion: that add rounds half to even, and the clamp never
  acts because |x| <= amax bounds the quotient by 127 (1 + 2^-23).

This checks both against IEEE single-precision division, rintf and the clamp, with gcc's
correctly rounded ``fmaf`` on the scales the kernels produce (s = amax/127 + 1e-7, |x| <= amax):
random elements, elements within a few ulps of half-integers (where a one-ulp quotient error
would flip the code), x = +-amax (the largest quotients), and the infinite-scale case.
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

SOURCE = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
static uint64_t st = 0x9E3779B97F4A7C15ull;
static inline uint64_t rnd(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return st; }
static inline float u01(void) { return (float)((rnd() >> 40) * (1.0 / 16777216.0)); }
static inline float quotient(float x, float scale) {
  const float y = 1.0f / scale;
  const float s = isinf(scale) ? 0.0f : scale;
  const float q0 = x * y;
  const float r = fmaf(-s, q0, x);
  return fmaf(r, y, q0);
}
static inline float code(float q) { return fminf(fmaxf(rintf(q), -127.0f), 127.0f); }
static inline float code_magic(float q) {
  const float t = q + 12582912.0f;
  uint32_t bits;
  memcpy(&bits, &t, 4);
  return (float)(int8_t)(bits & 0xffu);
}
int main(void) {
  long n = 0, bad = 0, near = 0, edge = 0;
  for (long it = 0; it < 3000000L; ++it) {
    float amax = ldexpf(1.0f + u01(), (int)(rnd() % 44) - 26);
    if (rnd() % 3 == 0) amax = (float)((rnd() % 65504) + 1) / 64.0f;
    const float s = amax / 127.0f + 1e-7f;
    float x;
    switch (rnd() % 4) {
      case 0: x = amax * (2.0f * u01() - 1.0f); break;
      case 3: x = (rnd() & 1) ? amax : -amax; ++edge; break;
      case 1: {
        const float k = (float)((int)(rnd() % 255) - 127) + 0.5f;
        x = k * s;
        if (rnd() & 1) x = nextafterf(x, (rnd() & 1) ? INFINITY : -INFINITY);
        ++near;
        break;
      }
      default: {
        const float k = (float)((int)(rnd() % 255) - 127) + 0.5f;
        x = fmaf(k, s, ((int)(rnd() % 64) - 32) * ldexpf(s, -24));
        ++near;
      }
    }
    if (!(fabsf(x) <= amax)) continue;
    ++n;
    bad += code(quotient(x, s)) != code(x / s);
    bad += code_magic(quotient(x, s)) != code(x / s);
  }
  /* infinite scale (non-finite input): finite x -> signed zero quotient, infinite x -> NaN */
  const float inf = INFINITY;
  const float xs[4] = {1.5f, -3.0f, 0.0f, 65504.0f};
  for (int i = 0; i < 4; ++i) {
    const float a = quotient(xs[i], inf), b = xs[i] / inf;
    bad += memcmp(&a, &b, 4) != 0;
  }
  bad += !isnan(quotient(inf, inf));
  bad += code_magic(quotient(inf, inf)) != 0.0f; /* NaN quotient -> code 0 */
  printf("%ld %ld %ld %ld\n", n, near, edge, bad);
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_kernel_codes_match_ieee_division_rint_and_clamp(tmp_path: Path) -> None:
    src = tmp_path / "division_identity.c"
    exe = tmp_path / "division_identity"
    src.write_text(SOURCE)
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", str(src), "-o", str(exe), "-lm"], check=True)
    n, near, edge, bad = map(int, subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split())
    assert n > 2_000_000 and near > 1_000_000 and edge > 500_000
    assert bad == 0

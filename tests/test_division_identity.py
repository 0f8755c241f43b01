"""The codec's code test without a per-element division (``below_midpoint``,
``threshold_inclusive`` and ``y_threshold`` in csrc/rolaq_common.h): comparing
y = x - mean with the row's three FP64-derived float thresholds gives the same
code as comparing the correctly rounded quotient y / std with -t, 0 and t,
which is what the reference computes per element (mla_quant/oscar.py:135-140).
Checked in C against true IEEE division on seeded random (y, std) pairs over
the exponent ranges the codec meets (|y| across 1e-16..1e16, std in
1e-4..1e4), on the floats next to every threshold, and on signed zeros and
subnormal divisors, for the default Lloyd-Max threshold and thresholds with
even and odd significands (the tie rule)."""

import os
import shutil
import subprocess
import tempfile

import pytest

SRC = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
static uint64_t st = 0x9E3779B97F4A7C15ull;
static inline uint64_t xr(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return st; }
static inline float bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t ubits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
/* the device helpers, statement for statement */
static double below_midpoint(float th) {
  uint32_t b = ubits(th);
  uint32_t below = (b << 1) == 0 ? 0x80000001u : ((int32_t)b < 0 ? b + 1 : b - 1);
  return 0.5 * ((double)bits(below) + (double)th);
}
static int threshold_inclusive(float th) { return (ubits(th) & 1u) == 0; }
static float y_threshold(double s, double mu, int incl) {
  double p = s * mu;
  float y = (float)p;
  double yd = (double)y;
  if (incl ? !(yd < p) : !(yd <= p)) return y;
  uint32_t b = ubits(y);
  return bits((b << 1) == 0 ? 1u : ((int32_t)b < 0 ? b - 1 : b + 1));
}
static float T;
static double MLO, MZ, MHI;
static int ILO, IHI;
static long bad, n;
static void check(float y, float s) {
  float q = y / s;
  int ref = (q >= -T) + (q >= 0.0f) + (q >= T);
  double sd = (double)s;
  float ylo = y_threshold(sd, MLO, ILO), y0 = y_threshold(sd, MZ, 1), yhi = y_threshold(sd, MHI, IHI);
  int got = (y >= ylo) + (y >= y0) + (y >= yhi);
  bad += got != ref;
  ++n;
}
int main(void) {
  const float ts[4] = {0.9810652732849121f, 0.5f, bits(0x3f7fffffu), bits(0x3f800001u)};
  for (int ti = 0; ti < 4; ++ti) {
    T = ts[ti];
    MLO = below_midpoint(-T); MZ = below_midpoint(0.0f); MHI = below_midpoint(T);
    ILO = threshold_inclusive(-T); IHI = threshold_inclusive(T);
    for (long i = 0; i < 3000000L; ++i) {
      uint64_t r = xr();
      float y = bits((uint32_t)(r & 0x807FFFFFu) | ((uint32_t)(74 + (r >> 32) % 107) << 23));
      float s = bits((uint32_t)((r >> 23) & 0x007FFFFFu) | ((uint32_t)(113 + (r >> 48) % 27) << 23));
      check(y, s);
      /* the floats around each threshold of this divisor */
      float th[3] = {y_threshold((double)s, MLO, ILO), y_threshold((double)s, MZ, 1), y_threshold((double)s, MHI, IHI)};
      for (int j = 0; j < 3; ++j)
        for (int k = -2; k <= 2; ++k) {
          uint32_t u = ubits(th[j]);
          if ((u << 1) == 0) continue;
          check(bits(u + (uint32_t)k), s);
        }
      /* quotients near +-t: y = s * t perturbed by a few ulps */
      float d = s * T;
      uint32_t u = ubits(d) + (uint32_t)(r % 9) - 4u;
      check(bits(u), s);
      check(-bits(u), s);
    }
    /* signed zeros, subnormal and extreme divisors */
    const float zs[6] = {0.0f, -0.0f, bits(1u), bits(0x80000001u), bits(0x00800000u), bits(0x80800000u)};
    for (long i = 0; i < 200000L; ++i) {
      uint64_t r = xr();
      float s = bits((uint32_t)(r & 0x007FFFFFu) | ((uint32_t)(1 + (r >> 32) % 253) << 23));
      for (int j = 0; j < 6; ++j) check(zs[j], s);
      check(bits((uint32_t)(r >> 32) & 0x807FFFFFu), s);
    }
  }
  printf("%ld %ld\n", bad, n);
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_threshold_codes_match_true_division():
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "q.c"), os.path.join(d, "q")
        with open(src, "w") as f:
            f.write(SRC)
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, src, "-lm"], check=True)
        bad, n = map(int, subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split())
    assert n > 150_000_000 and bad == 0


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_threshold_check_catches_a_wrong_rounding():
    """The check above fails when the helper rounds to nearest instead of up
    (a planted mistake in this copy of it, not in the library)."""
    planted = SRC.replace("if (incl ? !(yd < p) : !(yd <= p)) return y;", "return y;")
    assert planted != SRC
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "q.c"), os.path.join(d, "q")
        with open(src, "w") as f:
            f.write(planted)
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, src, "-lm"], check=True)
        bad, n = map(int, subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split())
    assert bad > 0

"""The writer's quotient: RN(q0 + r y), q0 = RN(d y), r = d - q0 s, y = RN(1 / s)
(``div_by`` in csrc/rolaq_common.h) equals the correctly rounded d / s, which
the reference computes per element (mla_quant/oscar.py:135). Checked in C with
hardware FMA on seeded random pairs over the exponent ranges the codec meets
(|x - mean| across 1e-16..1e16, std in 1e-4..1e4), plus edge patterns."""

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
static int check(float d, float s) {
  float y = 1.0f / s, q0 = d * y, q = fmaf(fmaf(-q0, s, d), y, q0), ref = d / s;
  return q == ref;
}
int main(void) {
  long bad = 0, n = 0;
  for (long i = 0; i < 20000000L; ++i) {
    uint64_t r = xr();
    float d = bits((uint32_t)(r & 0x807FFFFFu) | ((uint32_t)(74 + (r >> 32) % 107) << 23));
    float s = bits((uint32_t)((r >> 23) & 0x007FFFFFu) | ((uint32_t)(113 + (r >> 48) % 27) << 23));
    bad += !check(d, s);
    ++n;
  }
  /* quotients next to the Lloyd-Max threshold and 0: d = k * s * t near the boundary */
  const float t = 0.9810652732849121f;
  for (long i = 0; i < 2000000L; ++i) {
    uint64_t r = xr();
    float s = bits((uint32_t)((r >> 23) & 0x007FFFFFu) | ((uint32_t)(113 + (r >> 48) % 27) << 23));
    float d = s * t;
    uint32_t u; memcpy(&u, &d, 4); u += (uint32_t)(r % 9) - 4u; memcpy(&d, &u, 4);
    bad += !check(d, s) + !check(-d, s);
    n += 2;
  }
  printf("%ld %ld\n", bad, n);
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_fma_quotient_matches_true_division():
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "q.c"), os.path.join(d, "q")
        with open(src, "w") as f:
            f.write(SRC)
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, src, "-lm"], check=True)
        bad, n = map(int, subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split())
    assert n > 20_000_000 and bad == 0

"""The int8 activation rounding with one division per group (edgelm_amd/csrc/elm_quant.h) equals
edgelm's per-value division (quantize_act_row, kernels_ref.cpp:23-37) on every input checked:

* all non-negative floats up to 128 s (the reachable range |v| <= amax = 127 s, and past it), for
  two scales (the rounding is odd in v, so the sign is covered);
* for 20000 log-uniform random scales, the 64 floats around every rounding point (m - 1/2) s,
  m = 1 .. 127 (where a one-ulp quotient error would show), plus random values;
* scales outside the fast range, zero blocks and non-finite values.

The reference is the plain division compiled by gcc (IEEE single precision, no contraction).
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SRC = r"""
#include <math.h>
#include <stdio.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#define ELM_HOSTDEV
#include "elm_quant.h"
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static uint64_t rs = 88172645463325252ull;
static uint64_t rnd(void) { rs ^= rs << 13; rs ^= rs >> 7; rs ^= rs << 17; return rs; }
static unsigned long bad = 0, redo = 0, total = 0;
static void check4(const float* v, float safe) {
  int q[4];
  elm_q8_group<4>(v, safe, q);
  for (int i = 0; i < 4; ++i) {
    const int want = elm_q8_round(v[i] / safe);
    if (q[i] != want) {
      if (bad < 10) printf("MISMATCH v=%a safe=%a got %d want %d\n", v[i], safe, q[i], want);
      ++bad;
    }
  }
  total += 4;
}
int main(int argc, char** argv) {
  (void)argc; (void)argv;
  // 1. exhaustive over v in [0, 128 s] for a few scales
  const float scales[2] = {1.0f, 0x1.7c4a3ep-2f};
  for (int k = 0; k < 2; ++k) {
    const float s = scales[k];
    const uint32_t hi = f2u(128.0f * s);
    float v[4];
    int n = 0;
    for (uint32_t u = 0; u <= hi; ++u) {
      v[n++] = u2f(u);
      if (n == 4) { check4(v, s); n = 0; }
    }
  }
  // 2. random scales: every rounding point +- 32 ulp, and random values
  for (int k = 0; k < 20000; ++k) {
    const float amax = ldexpf(1.0f + (float)(rnd() % 1000000) / 1000000.0f, (int)(rnd() % 180) - 90);
    const float s = amax / 127.0f;
    const float safe = s == 0.f ? 1.f : s;
    float v[4];
    int n = 0;
    for (int m = 1; m <= 127; ++m) {
      const uint32_t c = f2u((m - 0.5f) * safe);
      for (int d = -32; d < 32; ++d) {
        float x = u2f(c + d);
        if (rnd() & 1) x = -x;
        if (fabsf(x) > amax) x = copysignf(amax, x);
        v[n++] = x;
        if (n == 4) { check4(v, safe); n = 0; }
      }
    }
    for (int i = 0; i < 64; ++i) {
      v[n++] = amax * ((float)(int64_t)(rnd() % 2000001) / 1000000.0f - 1.0f);
      if (n == 4) { check4(v, safe); n = 0; }
    }
  }
  // 3. edge scales and values
  const float edge_s[6] = {0x1p-126f, 0x1p-140f, 0x1p-101f, 0x1p101f, 0x1.fffffep127f, INFINITY};
  const float edge_v[8] = {0.f, -0.f, 1.0f, -3.5f, 0x1p-149f, NAN, INFINITY, -INFINITY};
  for (int k = 0; k < 6; ++k)
    for (int i = 0; i < 8; i += 4) check4(edge_v + i, edge_s[k]);
  float z[4] = {0.f, 0.f, -0.f, 0.f};
  check4(z, 1.0f);
  printf("%lu %lu\n", bad, total);
  return bad != 0;
}
"""


def test_group_rounding_equals_division(tmp_path):
    src = tmp_path / "q8_check.cpp"
    src.write_text(SRC)
    exe = tmp_path / "q8_check"
    subprocess.run(["g++", "-O2", "-ffp-contract=off", "-Wno-unknown-pragmas", "-I",
                    os.path.join(ROOT, "edgelm_amd", "csrc"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=900)
    assert out.returncode == 0, out.stdout[-2000:]
    bad, total = map(int, out.stdout.split()[-2:])
    assert bad == 0 and total > 2_000_000_000

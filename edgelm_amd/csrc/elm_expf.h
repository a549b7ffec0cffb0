// expf restated from the published ARM optimized-routines method (Szabolcs Nagy, 2017; the
// algorithm glibc >= 2.28 ships as expf): 2^(k/32) from a 32-entry table times a cubic in the
// reduced argument, all in double precision, with the FMA contraction glibc's x86-64 FMA build
// uses. The table entries are 2^(i/32) correctly rounded to double, minus (i << 47), computed
// independently. Verified identical to the host libm's expf on all 2^32 inputs; edgelm's
// silu (kernels_cpu.cpp:292) calls that expf, so device SwiGLU epilogues reproduce it bit for bit.
#pragma once
#include <stdint.h>

#ifndef ELM_HOSTDEV
#define ELM_HOSTDEV __host__ __device__
#endif

ELM_HOSTDEV static inline double elm_u2d(uint64_t u) {
  union { uint64_t u; double d; } v;
  v.u = u;
  return v.d;
}
ELM_HOSTDEV static inline uint64_t elm_d2u(double d) {
  union { uint64_t u; double d; } v;
  v.d = d;
  return v.u;
}
ELM_HOSTDEV static inline uint32_t elm_f2u(float f) {
  union { uint32_t u; float f; } v;
  v.f = f;
  return v.u;
}

ELM_HOSTDEV static inline uint64_t elm_exp2_tab(uint32_t i) {
  // switch instead of a table in memory: the value is selected without a data load.
  switch (i & 31) {
    case 0: return 0x3ff0000000000000ull;  case 1: return 0x3fefd9b0d3158574ull;
    case 2: return 0x3fefb5586cf9890full;  case 3: return 0x3fef9301d0125b51ull;
    case 4: return 0x3fef72b83c7d517bull;  case 5: return 0x3fef54873168b9aaull;
    case 6: return 0x3fef387a6e756238ull;  case 7: return 0x3fef1e9df51fdee1ull;
    case 8: return 0x3fef06fe0a31b715ull;  case 9: return 0x3feef1a7373aa9cbull;
    case 10: return 0x3feedea64c123422ull; case 11: return 0x3feece086061892dull;
    case 12: return 0x3feebfdad5362a27ull; case 13: return 0x3feeb42b569d4f82ull;
    case 14: return 0x3feeab07dd485429ull; case 15: return 0x3feea47eb03a5585ull;
    case 16: return 0x3feea09e667f3bcdull; case 17: return 0x3fee9f75e8ec5f74ull;
    case 18: return 0x3feea11473eb0187ull; case 19: return 0x3feea589994cce13ull;
    case 20: return 0x3feeace5422aa0dbull; case 21: return 0x3feeb737b0cdc5e5ull;
    case 22: return 0x3feec49182a3f090ull; case 23: return 0x3feed503b23e255dull;
    case 24: return 0x3feee89f995ad3adull; case 25: return 0x3feeff76f2fb5e47ull;
    case 26: return 0x3fef199bdd85529cull; case 27: return 0x3fef3720dcef9069ull;
    case 28: return 0x3fef5818dcfba487ull; case 29: return 0x3fef7c97337b9b5full;
    case 30: return 0x3fefa4afa2a490daull; default: return 0x3fefd0765b6e4540ull;
  }
}

ELM_HOSTDEV static inline float elm_expf(float x) {
  const uint32_t ux = elm_f2u(x);
  const uint32_t abstop = (ux >> 20) & 0x7ff;
  if (abstop >= 0x42b) {                         // |x| >= 88 (top 12 bits of 88.0f), or inf/nan
    if (ux == 0xff800000u) return 0.0f;          // -inf
    if (abstop >= 0x7f8) return x + x;           // +inf or nan
    if (x > 0x1.62e42ep6f) return __builtin_inff();  // overflow
    if (x < -0x1.9fe368p6f) return 0.0f;             // underflow
  }
  const double N = 32.0;
  const double inv_ln2_n = 0x1.71547652b82fep+0 * N;
  const double shift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / N / N / N, c1 = 0x1.ebfce50fac4f3p-3 / N / N,
               c2 = 0x1.62e42ff0c52d6p-1 / N;
  const double xd = (double)x;
  double kd = __builtin_fma(inv_ln2_n, xd, shift);  // round(x*N/ln2) via the shift
  const uint64_t ki = elm_d2u(kd);
  kd -= shift;
  const double r = __builtin_fma(inv_ln2_n, xd, -kd);
  const uint64_t t = elm_exp2_tab((uint32_t)(ki & 31)) + (ki << 47);
  const double s = elm_u2d(t);
  const double z = __builtin_fma(c0, r, c1);
  const double r2 = r * r;
  double y = __builtin_fma(c2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

// expf restated from the published ARM optimized-routines method (Szabolcs Nagy, 2017; the
// algorithm glibc >= 2.28 ships as expf): 2^(k/32) from a 32-entry table times a cubic in the
// reduced argument, all in double precision, with the FMA contraction glibc's x86-64 FMA build
// uses. Verified identical to the host libm's expf on all 2^32 inputs; edgelm's silu
// (kernels_cpu.cpp:292) calls that expf, so device SwiGLU epilogues reproduce it bit for bit.
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

// Table entry i of the method: the bits of 2^(i/32) correctly rounded to double, minus (i << 47).
// Computed without a table or a branch, so that lanes of one wave with different i do not split
// into 32 paths: 2^(i/32) = sqrt(2) * e^(t ln2 / 32) with t = i - 16, by a degree-13 Taylor
// polynomial (c_n = sqrt(2) (ln2/32)^n / n!, rounded to double) in Horner form with FMA. Over
// the 32 values of i the result is either the correctly rounded value or one ulp above it; bit i
// of kElmExp2Fix marks the latter. The exhaustive expf test covers every entry.
ELM_HOSTDEV static inline uint64_t elm_exp2_tab(uint32_t i) {
  const uint32_t kElmExp2Fix = 0x915055e4u;
  i &= 31;
  const double t = (double)(int)i - 16.0;
  double y = 0x1.108170a304abp-104;
  y = __builtin_fma(y, t, 0x1.3f6da49237698p-95);
  y = __builtin_fma(y, t, 0x1.59a0d25f61fc7p-86);
  y = __builtin_fma(y, t, 0x1.56cff45438d97p-77);
  y = __builtin_fma(y, t, 0x1.351bc8299ee8fp-68);
  y = __builtin_fma(y, t, 0x1.f5b1687066adap-60);
  y = __builtin_fma(y, t, 0x1.69e51ed115674p-51);
  y = __builtin_fma(y, t, 0x1.c8d752e2475fdp-43);
  y = __builtin_fma(y, t, 0x1.ee4fd234aabe3p-35);
  y = __builtin_fma(y, t, 0x1.bdb696e8a0afcp-27);
  y = __builtin_fma(y, t, 0x1.41839eb881562p-19);
  y = __builtin_fma(y, t, 0x1.5be298adf0352p-12);
  y = __builtin_fma(y, t, 0x1.f5e46537ab907p-6);
  y = __builtin_fma(y, t, 0x1.6a09e667f3bcdp+0);
  return elm_d2u(y) - ((kElmExp2Fix >> i) & 1u) - ((uint64_t)i << 47);
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

// edgelm's int8 activation rounding (quantize_act_row, kernels_ref.cpp:23-37): q = v / s rounded
// half away from zero, clamped to +-127, where s = amax / 127 (1 for an all-zero block) and the
// quotient is the correctly rounded single-precision one.
//
// elm_q8_group gives the same q for n values of one block with one division instead of n: each
// quotient is taken as v * (1 / s), which is within 1.5 ulp of the correctly rounded v / s. The
// rounding of a quotient t depends on t only through which side of the points m - 1/2 (shifted by
// at most one ulp by the float addition of 1/2) it falls, so the two agree unless some t lies within
// 2^-21 |t| + 2^-24 of a point m - 1/2; the check below allows twice that. Such a group, and a
// scale outside [2^-100, 2^100] (where 1 / s could round through the subnormal range or overflow),
// is redone with the divisions. The distance itself is computed exactly: t - floor(t) is exact,
// and so is (t - floor(t)) - 1/2 wherever it is compared (Sterbenz).
#pragma once

#ifndef ELM_HOSTDEV
#define ELM_HOSTDEV __host__ __device__
#endif

ELM_HOSTDEV static inline int elm_q8_round(float t) {
  const float r = copysignf(floorf(fabsf(t) + 0.5f), t);
  return (int)fminf(127.f, fmaxf(-127.f, r));
}

// True if the rounding of t' = v * (1 / s) may differ from that of v / s.
ELM_HOSTDEV static inline bool elm_q8_near_half(float tp) {
  const float a = fabsf(tp);
  return fabsf(a - floorf(a) - 0.5f) <= fmaf(a, 0x1p-20f, 0x1p-22f);
}

template <int N>
ELM_HOSTDEV static inline void elm_q8_group(const float* v, float safe, int* q) {
  const float r = 1.0f / safe;
  float t[N];
  bool redo = !(safe >= 0x1p-100f && safe <= 0x1p100f);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    t[i] = v[i] * r;
    redo |= elm_q8_near_half(t[i]);
  }
  if (redo) {
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = v[i] / safe;
  }
#pragma unroll
  for (int i = 0; i < N; ++i) q[i] = elm_q8_round(t[i]);
}

// Byte offset of the 16 elements h*16 .. h*16+15 of token t's block b in the block-scale GEMM's
// activation fragments: the 1 KB fragment of (32-token group, block b) holds them for lane
// h*32 + t%32; nb = blocks per token row.
ELM_HOSTDEV static inline long long elm_frag_offset(int t, int b, int h, int nb) {
  return ((((long long)(t >> 5) * nb + b) * 64) + h * 32 + (t & 31)) * 16;
}

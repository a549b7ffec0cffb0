// Device helpers of the int8 GEMVs: edgelm's activation rounding for one 32-block held by 8 lanes, the
// exact int8 item product of q8 / q4 weights, and the block-order fold of a row of products
// (kernels_cpu.cpp:159-167,193-204: sequential adds, multiply and add rounded separately).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "elm_dpp.h"
#include "elm_expf.h"
#include "elm_quant.h"
#include "elmh_internal.hpp"

namespace elmh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float silu_exact(float v) { return v / (1.0f + elm_expf(-v)); }

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Quantizes one 32-value block held by 8 consecutive lanes (lanes 8k .. 8k+7 of a wave, 4 values
// each, in order); every lane of the group gets the block scale (returned) and the block sum of q.
// Same arithmetic as quantize_act_row (kernels_ref.cpp:23-37): the amax is order-free, the
// rounding of every value that of its division (elm_q8_group). Every lane of the wave must run it.
__device__ __forceinline__ float quant_block8x4(const float (&v)[4], int (&q)[4], int& sum) {
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) a = fmaxf(a, fabsf(v[i]));
  a = fmaxf(a, dpp_f<kDppQuadXor1>(a));
  a = fmaxf(a, dpp_f<kDppQuadXor2>(a));
  a = fmaxf(a, dpp_f<kDppHalfMirror>(a));
  const float s = a / 127.0f;
  elm_q8_group<4>(v, s == 0.f ? 1.f : s, q);
  int sm = q[0] + q[1] + q[2] + q[3];
  sm += dpp_i<kDppQuadXor1>(sm);
  sm += dpp_i<kDppQuadXor2>(sm);
  sm += dpp_i<kDppHalfMirror>(sm);
  sum = sm;
  return s;
}

__device__ __forceinline__ uint32_t pack_q4(const int (&q)[4]) {
  return (uint32_t)(q[0] & 0xFF) | (uint32_t)(q[1] & 0xFF) << 8 | (uint32_t)(q[2] & 0xFF) << 16 |
         (uint32_t)(q[3] & 0xFF) << 24;
}

__device__ __forceinline__ int fold_stride(int nb) {
  const int p = (nb + 3) & ~3;
  return ((p >> 2) & 1) ? p : p + 4;  // multiple of 4 (16-byte rows), odd in float4 units
}

template <int WDT>
__device__ __forceinline__ float item_product(const v4u w0, const v4u w1, float wsc, const int8_t* act, float xd,
                                              int xs) {
  const int4* aq = reinterpret_cast<const int4*>(act);
  const int4 a0 = aq[0], a1 = aq[1];
  if (WDT == WQ8) {
    int S = sdot4((int)w0.x, a0.x, 0);
    S = sdot4((int)w0.y, a0.y, S);
    S = sdot4((int)w0.z, a0.z, S);
    S = sdot4((int)w0.w, a0.w, S);
    S = sdot4((int)w1.x, a1.x, S);
    S = sdot4((int)w1.y, a1.y, S);
    S = sdot4((int)w1.z, a1.z, S);
    S = sdot4((int)w1.w, a1.w, S);
    return (float)S * xd;
  }
  // sum_i (nib_i - 8) x_i = sum_i nib_i x_i - 8 * sum_i x_i (nibbles 0..15 are valid int8)
  int S = -8 * xs;
  S = sdot4((int)(w0.x & 0x0F0F0F0Fu), a0.x, S);
  S = sdot4((int)(w0.y & 0x0F0F0F0Fu), a0.y, S);
  S = sdot4((int)(w0.z & 0x0F0F0F0Fu), a0.z, S);
  S = sdot4((int)(w0.w & 0x0F0F0F0Fu), a0.w, S);
  S = sdot4((int)((w0.x >> 4) & 0x0F0F0F0Fu), a1.x, S);
  S = sdot4((int)((w0.y >> 4) & 0x0F0F0F0Fu), a1.y, S);
  S = sdot4((int)((w0.z >> 4) & 0x0F0F0F0Fu), a1.z, S);
  S = sdot4((int)((w0.w >> 4) & 0x0F0F0F0Fu), a1.w, S);
  return (float)S * (wsc * xd);
}

// Four block-order adds into one accumulator (no reassociation).
__device__ __forceinline__ void add4(float& acc, const float4 v) {
  acc = acc + v.x;
  acc = acc + v.y;
  acc = acc + v.z;
  acc = acc + v.w;
}

// Block-order fold of one LDS row of nb products into one accumulator. A wave issues one vector
// instruction every few cycles and the fold runs on few waves, so the code keeps its instruction
// count low: whole float4 are read eight at a time before the first add, the rest of the row (up
// to seven float4 and the last nb % 4 values) in one more batch, and every branch depends on nb
// only (uniform, no lane masking). Reads past the row's last whole float4 are clamped into the row.
__device__ __forceinline__ float fold_chain(const float* row, int nb) {
  const float4* p4 = reinterpret_cast<const float4*>(row);
  const int nq = nb >> 2;
  float acc = 0.f;
  int q0 = 0;
  for (; q0 + 8 <= nq; q0 += 8) {
    float4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = p4[q0 + i];
#pragma unroll
    for (int i = 0; i < 8; ++i) add4(acc, v[i]);
  }
  const int nr = nq - q0;  // 0 .. 7
  float4 v[7];
#pragma unroll
  for (int i = 0; i < 7; ++i) v[i] = p4[q0 + min(i, max(nr - 1, 0))];
  const float4 t = p4[(nb - 1) >> 2];  // holds the last nb % 4 values
#pragma unroll
  for (int i = 0; i < 7; ++i)
    if (i < nr) add4(acc, v[i]);
  const int nt = nb & 3;
  if (nt > 0) acc = acc + t.x;
  if (nt > 1) acc = acc + t.y;
  if (nt > 2) acc = acc + t.z;
  return acc;
}

// Value of lane (i + 8) mod 16 within each 16-lane row of the wave (DPP row rotate by 8): swaps
// the two halves of every row in one VALU instruction.
__device__ __forceinline__ float row_swap8(float v) {
  return dpp_f<kDppRowRor8>(v);
}

}  // namespace
}  // namespace elmh

// In-order float sums read from LDS, for the kernels of both device sources: edgelm's sequential
// accumulations (the RMSNORM sums of squares, the softmax denominator) as straight-line code that
// reads ahead, so the dependent adds wait for LDS once per batch.
#pragma once
#include <hip/hip_runtime.h>

namespace elmh {

// acc + x_0 + x_1 + ... + x_{16 nbt - 1} in order (nbt <= 16), x_k = row[k]; all 256 values of
// the row lie in LDS (those past 16 nbt are read ahead but never added). Straight-line code over
// batches of 16: batch b + 2 is read before batch b is added, and every read is unconditional
// once its step is reached (the empty asm keeps the compiler from sinking it past the exits), so
// the wait before a batch's adds covers that batch only. (A loop with the same reads ahead waits
// for every read at its head: the compiler's wait-count pass merges the exit path's state.)
__device__ __forceinline__ float ordered_sum256(const float* __restrict__ row, int nbt, float acc) {
  float4 b[3][4];
#define ELM_SUM_LOAD(bt)                                                                           \
  _Pragma("unroll") for (int u = 0; u < 4; ++u) b[(bt) % 3][u] =                                   \
      *reinterpret_cast<const float4*>(row + 16 * (bt) + 4 * u);                                   \
  asm volatile("" ::: "memory");
#define ELM_SUM_STEP(bt)                                                                           \
  if (nbt <= (bt)) goto done;                                                                      \
  if ((bt) + 2 < 16) { ELM_SUM_LOAD((bt) + 2) }                                                    \
  _Pragma("unroll") for (int u = 0; u < 4; ++u) {                                                  \
    acc = acc + b[(bt) % 3][u].x;                                                                  \
    acc = acc + b[(bt) % 3][u].y;                                                                  \
    acc = acc + b[(bt) % 3][u].z;                                                                  \
    acc = acc + b[(bt) % 3][u].w;                                                                  \
  }
  ELM_SUM_LOAD(0)
  ELM_SUM_LOAD(1)
  ELM_SUM_STEP(0) ELM_SUM_STEP(1) ELM_SUM_STEP(2) ELM_SUM_STEP(3) ELM_SUM_STEP(4) ELM_SUM_STEP(5)
  ELM_SUM_STEP(6) ELM_SUM_STEP(7) ELM_SUM_STEP(8) ELM_SUM_STEP(9) ELM_SUM_STEP(10) ELM_SUM_STEP(11)
  ELM_SUM_STEP(12) ELM_SUM_STEP(13) ELM_SUM_STEP(14) ELM_SUM_STEP(15)
#undef ELM_SUM_STEP
#undef ELM_SUM_LOAD
done:
  return acc;
}

// Length of a row of squares in LDS for an in-order sum of K/4 values through ordered_sum256: the
// values rounded up to whole batches of 16 (the padding holds +0.0, which changes no sum of squares)
// and two more batches that the reads ahead may touch.
__host__ __device__ inline int norm_rowlen(int K) { return (((K >> 2) + 15) / 16 + 2) * 16; }

// acc + row[0] + ... + row[n - 1] in order, for any n, through ordered_sum256 256 values at a time; the
// caller pads [n, 16 ceil(n / 16)) with +0.0 and keeps two more batches of 16 readable (norm_rowlen)
__device__ __forceinline__ float ordered_sum(const float* __restrict__ row, int n, float acc) {
  const int nbt = (n + 15) >> 4;
  for (int g0 = 0; g0 < nbt; g0 += 16) acc = ordered_sum256(row + 16 * g0, min(16, nbt - g0), acc);
  return acc;
}

}  // namespace elmh

// Cross-lane moves within a wave in one VALU instruction (DPP, gfx9 encodings), for the kernels
// of both device sources.
#pragma once
#include <hip/hip_runtime.h>

namespace elmh {

// quad_perm [1,0,3,2] (swap neighbours), quad_perm [2,3,0,1] (swap pairs), row_half_mirror
// (lane i <- 7 - i within each 8 lanes), row_mirror (lane i <- 15 - i within each 16 lanes),
// row_ror:8 (lane i <- (i + 8) mod 16 within each 16 lanes)
constexpr int kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppHalfMirror = 0x141, kDppRowMirror = 0x140,
              kDppRowRor8 = 0x128;

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}

// fmaxf over the 64 lanes of the wave (every lane active); the result is wave-uniform. The order
// of the steps does not change the result: fmaxf ignores a NaN operand, and the maximum of the
// other values is unique but for the sign of a zero.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppRowMirror>(v));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Integer sum over the 64 lanes of the wave (every lane active); the result is wave-uniform (an
// integer sum does not depend on its order).
__device__ __forceinline__ int wave_sum_i(int v) {
  v += dpp_i<kDppQuadXor1>(v);
  v += dpp_i<kDppQuadXor2>(v);
  v += dpp_i<kDppHalfMirror>(v);
  v += dpp_i<kDppRowMirror>(v);
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
         __builtin_amdgcn_readlane(v, 48);
}

}  // namespace elmh

// HIP kernels (gfx950) for edgelm's quantized-matmul family: MATMUL / MATMUL_N / MATMUL_ADD /
// FFN_SWIGLU with q8 per-row or q4 group-32 weights and f32 or dynamic int8 activations.
//
// Numerics follow edgelm's cpu backend on its scalar path bit for bit:
//  * int8 activations (kernels_ref.cpp:23-37): per row, per 32-block amax/127, IEEE divide,
//    round half away from zero, clamp +-127 (one division per lane group, elm_quant.h);
//  * int8 block sums S_b are exact int32 dot products (v_dot4 / MFMA), order-free;
//  * the f32 fold over blocks is sequential in block order with separate multiply and add
//    (kernels_cpu.cpp:159-167, 193-204; this file is compiled with -ffp-contract=off and every
//    fused multiply-add below is explicit);
//  * f32-activation paths keep the scalar path's four interleaved accumulators
//    (kernels_cpu.cpp:32-43, 45-71) and per-group order (73-112);
//  * silu uses an expf identical to the host libm's (elm_expf.h).
#include "elm_dpp.h"
#include "elm_expf.h"
#include "elm_quant.h"
#include "elmh_internal.hpp"
#include "elm_gemv.h"
#include "elm_dma.h"
#include "elm_sum.h"

#include <cstring>

namespace elmh {
namespace {

// q4 group bytes -> MFMA int8 operand for half h: 16*q of elements h*16 .. h*16+15
// (low nibbles for h = 0, high for h = 1). x ^ 8 maps the stored q+8 to q's 4-bit two's
// complement; placed in the high nibble of a byte it reads as 16*q.
__device__ __forceinline__ v4i q4_operand16(uint4 w, int h) {
  const int sh = 4 - 4 * h;
  v4i r;
  r.x = (int)(((w.x << sh) & 0xF0F0F0F0u) ^ 0x80808080u);
  r.y = (int)(((w.y << sh) & 0xF0F0F0F0u) ^ 0x80808080u);
  r.z = (int)(((w.z << sh) & 0xF0F0F0F0u) ^ 0x80808080u);
  r.w = (int)(((w.w << sh) & 0xF0F0F0F0u) ^ 0x80808080u);
  return r;
}

// ---------------------------------------------------------------- weight repack

__global__ void repack_kernel(const uint8_t* __restrict__ raw, const float* __restrict__ raw_scales,
                              uint8_t* __restrict__ out, float* __restrict__ out_scales, int64_t rows, int64_t cols,
                              int64_t nb, int64_t rows_pad, int H, int dtype) {
  const int64_t items = rows_pad * nb;
  const int G = dtype == WQ8 ? 32 : 16;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < items; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i / nb, b = i - n * nb;
    const int64_t dst = item_index(n, b, nb, H);
    uint8_t* o = out + dst * G;
    if (dtype == WQ8) {
      for (int j = 0; j < 32; ++j) {
        const int64_t k = b * 32 + j;
        o[j] = (n < rows && k < cols) ? raw[n * cols + k] : 0;
      }
    } else {
      for (int j = 0; j < 16; ++j) o[j] = n < rows ? raw[n * (cols / 2) + b * 16 + j] : 0x88;  // 0x88: q = 0
      out_scales[dst] = n < rows ? raw_scales[n * nb + b] : 0.f;
    }
  }
  if (dtype == WQ8)
    for (int64_t n = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; n < rows_pad; n += (int64_t)gridDim.x * blockDim.x)
      out_scales[n] = n < rows ? raw_scales[n] : 0.f;
}

// ---------------------------------------------------------------- activation quantization

// Row-major: 32 blocks per 256-thread workgroup, 4 values per thread (8 threads per block).
__global__ __launch_bounds__(256) void act_quant_rows_kernel(const float* __restrict__ x, int T, int K,
                                                             int8_t* __restrict__ xq, float* __restrict__ xd,
                                                             int32_t* __restrict__ xs) {
  // every argument in scalar registers first, through one statement: their loads go out together and
  // the arithmetic on T and K waits for the statement (one round trip to the argument segment)
  asm volatile("" : "+s"(T), "+s"(K) : "s"(x), "s"(xq), "s"(xd), "s"(xs));
  const int nb = K / kBlock;
  const int g = blockIdx.x * 32 + (threadIdx.x >> 3), l = (threadIdx.x & 7) * 4;
  const bool ok = g < T * nb;
  const int t = ok ? g / nb : 0, b = ok ? g - t * nb : 0;
  const int64_t e = (int64_t)t * K + b * kBlock + l;
  // four scalar loads the compiler merges into one 16-byte load (x need only be 4-byte aligned)
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (ok)
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = x[e + i];
  int q[4], sum;
  const float d = quant_block8x4(v, q, sum);
  if (!ok) return;
  *reinterpret_cast<uint32_t*>(xq + e) = pack_q4(q);
  if (l == 0) {
    xd[(int64_t)t * nb + b] = d;
    xs[(int64_t)t * nb + b] = sum;
  }
}

// Fragment-major for the MFMA GEMM: the 1 KB fragment of (32-token group, block b) holds for lane
// L = h*32 + t%32 the 16 bytes of elements h*16 .. h*16+15 of token t's block b. A thread owns one
// such half-block: four float4 loads, edgelm's rounding, one 16-byte store.

// edgelm's rounding of v / safe (quantize_act_row, kernels_ref.cpp:23-37) for 16 values of one
// block, packed in order (elm_q8_group: one division for the 16)
__device__ __forceinline__ uint4 q8x16(const float4 (&v)[4], float safe) {
  const float f[16] = {v[0].x, v[0].y, v[0].z, v[0].w, v[1].x, v[1].y, v[1].z, v[1].w,
                       v[2].x, v[2].y, v[2].z, v[2].w, v[3].x, v[3].y, v[3].z, v[3].w};
  int q[16];
  elm_q8_group<16>(f, safe, q);
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = pack_q4({q[4 * i], q[4 * i + 1], q[4 * i + 2], q[4 * i + 3]});
  return make_uint4(w[0], w[1], w[2], w[3]);
}
__device__ __forceinline__ float amax4(float4 v, float a) {
  return fmaxf(fmaxf(fmaxf(a, fabsf(v.x)), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}
// floats 4i .. 4i+3 of p; the compiler merges these into 16-byte loads, which the hardware serves
// at any 4-byte alignment (x may point anywhere into a caller's tensor)
__device__ __forceinline__ float4 ld4(const float* p, int i) {
  return make_float4(p[4 * i], p[4 * i + 1], p[4 * i + 2], p[4 * i + 3]);
}
__device__ __forceinline__ int64_t frag_offset(int t, int b, int h, int nb) { return elm_frag_offset(t, b, h, nb); }

// Per-32-block scales. Workgroup = (32-token group g, blocks 4 y .. 4 y + 3); wave w takes block
// b = 4 y + w and lane L = h*32 + t%32 the 16 elements of half h of token t's block b, so each wave
// writes one whole 1 KB fragment; the block scale comes from the amax of lanes L and L ^ 32.
__global__ __launch_bounds__(256) void act_quant_frag_kernel(const float* __restrict__ x, int T, int Tpad, int K,
                                                             int8_t* __restrict__ xq, float* __restrict__ xd) {
  // every argument in scalar registers first, through one statement (as act_quant_rows_kernel)
  asm volatile("" : "+s"(T), "+s"(Tpad), "+s"(K) : "s"(x), "s"(xq), "s"(xd));
  const int nb = K / kBlock, g = blockIdx.x, lane = threadIdx.x & 63;
  const int b = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (b >= nb) return;  // whole waves
  const int h = lane >> 5, t = g * 32 + (lane & 31);
  const bool ok = t < T;
  const float* src = x + (int64_t)t * K + b * kBlock + h * 16;
  float4 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = ok ? ld4(src, i) : make_float4(0.f, 0.f, 0.f, 0.f);
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) a = amax4(v[i], a);
  a = fmaxf(a, __shfl_xor(a, 32, 64));
  const float sc = a / 127.0f;
  const float safe = sc == 0.f ? 1.f : sc;
  *reinterpret_cast<uint4*>(xq + ((int64_t)(g * nb + b) * 64 + lane) * 16) =
      q8x16(v, safe);
  if (h == 0) xd[(int64_t)b * Tpad + t] = sc;
}

// RMSNORM and the GEMM's per-block activation quantization in one pass (the input of a layer's
// QKV and gate/up GEMMs): kNqTok rows per workgroup, each normalized in rmsnorm_kernel's order
// (squares grouped by dot_f32_scalar's accumulators in LDS, four in-order sums, (s0 + s1) +
// (s2 + s3), then (x * inv) * w), then quantized into fragments exactly as act_quant_frag_kernel
// does. A thread owns up to kNqItems half-blocks (row, block, half) and loads their x and norm
// weights at the start, so the normalized values never leave its registers; the two halves of a
// block sit in neighbouring lanes. Tokens at or past T give zero fragments and scales. K <= 2048.
constexpr int kNqTok = 4;
constexpr int kNqItems = 2;  // kNqTok * (2048 / 32) * 2 half-blocks over 256 threads

__global__ __launch_bounds__(256) void rmsnorm_quant_frag_kernel(const float* __restrict__ x, const float* __restrict__ nw,
                                                                 float eps, int T, int Tpad, int K,
                                                                 int8_t* __restrict__ xq, float* __restrict__ xd) {
  extern __shared__ __align__(16) float nq_lds[];
  __shared__ float inv_l[kNqTok];
  const int K4 = K >> 2, rowlen = norm_rowlen(K), nb = K / kBlock;
  float* sq = nq_lds;  // [kNqTok][4][rowlen]
  const int t0 = blockIdx.x * kNqTok, tid = threadIdx.x, items = kNqTok * nb * 2;
  float4 xv[kNqItems][4], wv[kNqItems][4];
#pragma unroll
  for (int i = 0; i < kNqItems; ++i) {
    const int it = tid + 256 * i;
    const int r = it / (2 * nb), rem = it - r * 2 * nb, t = t0 + r;
    const int e0 = (rem >> 1) * kBlock + (rem & 1) * 16;  // first element of the half-block
    const bool in = it < items, ld = in && t < T;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xv[i][j] = ld ? ld4(x + (int64_t)t * K + e0, j) : make_float4(0.f, 0.f, 0.f, 0.f);
      wv[i][j] = in ? ld4(nw + e0, j) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (in) {
      float* q = sq + r * 4 * rowlen + (e0 >> 2);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        q[j] = xv[i][j].x * xv[i][j].x;
        q[rowlen + j] = xv[i][j].y * xv[i][j].y;
        q[2 * rowlen + j] = xv[i][j].z * xv[i][j].z;
        q[3 * rowlen + j] = xv[i][j].w * xv[i][j].w;
      }
    }
  }
  // +0.0 up to the next multiple of 16 terms
  for (int i = tid; i < kNqTok * 4 * 16; i += 256)
    if (K4 + (i & 15) < ((K4 + 15) & ~15)) sq[(i >> 4) * rowlen + K4 + (i & 15)] = 0.f;
  __syncthreads();
  if (tid < 4 * kNqTok) {
    const float sacc = ordered_sum(sq + tid * rowlen, K4, 0.f);
    const float s01 = sacc + dpp_f<kDppQuadXor1>(sacc);
    const float ss = s01 + dpp_f<kDppQuadXor2>(s01);
    if ((tid & 3) == 0) inv_l[tid >> 2] = 1.0f / sqrtf(ss / (float)K + eps);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kNqItems; ++i) {
    const int it = tid + 256 * i;
    if (it < items) {  // items is even: both lanes of a block pair take this branch
      const int r = it / (2 * nb), rem = it - r * 2 * nb, b = rem >> 1, h = rem & 1, t = t0 + r;
      const float inv = inv_l[r];
      float4 v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        v[j] = make_float4((xv[i][j].x * inv) * wv[i][j].x, (xv[i][j].y * inv) * wv[i][j].y,
                           (xv[i][j].z * inv) * wv[i][j].z, (xv[i][j].w * inv) * wv[i][j].w);
      float a = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) a = amax4(v[j], a);
      a = fmaxf(a, dpp_f<kDppQuadXor1>(a));
      const float sc = a / 127.0f;
      *reinterpret_cast<uint4*>(xq + frag_offset(t, b, h, nb)) = q8x16(v, sc == 0.f ? 1.f : sc);
      if (h == 0) xd[(int64_t)b * Tpad + t] = sc;
    }
  }
}

// Per-token scale (extension): one workgroup per token row. NF > 0: thread tid keeps the row's
// float4s f = tid + 256 i (i < NF; K <= 1024 NF) in registers between the row amax and the rounding,
// so each load instruction of a wave reads 1 KB of consecutive floats, and four consecutive lanes
// write a half-block's 16 bytes (the rounding of a value does not depend on its group: elm_q8_group
// of 4 gives the same q as of 16). NF == 0 reads the row twice, the second time from cache.
template <int NF>
__global__ __launch_bounds__(256) void act_quant_frag_token_kernel(const float* __restrict__ x, int T, int Tpad, int K,
                                                                   int8_t* __restrict__ xq, float* __restrict__ xd) {
  asm volatile("" ::"s"(x), "s"(T), "s"(Tpad), "s"(K), "s"(xq), "s"(xd));
  __shared__ float red[4];
  const int t = blockIdx.x, nb = K / kBlock, hb = 2 * nb, K4 = K >> 2;
  const float* row = x + (int64_t)t * K;
  constexpr int NR = NF > 0 ? NF : 1;
  float4 v[NR];
  float a = 0.f;
  if (NF > 0) {
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int f = threadIdx.x + 256 * i;
      v[i] = t < T && f < K4 ? ld4(row + 4 * f, 0) : make_float4(0.f, 0.f, 0.f, 0.f);
      a = amax4(v[i], a);
    }
  } else if (t < T) {
    for (int j = threadIdx.x; j < hb; j += 256) {
#pragma unroll
      for (int u = 0; u < 4; ++u) a = amax4(ld4(row + j * 16, u), a);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = a;
  __syncthreads();
  a = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = a / 127.0f;
  const float safe = sc == 0.f ? 1.f : sc;
  if (NF > 0) {
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int f = threadIdx.x + 256 * i, j = f >> 2;
      if (f < K4) {
        const float fv[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
        int q[4];
        elm_q8_group<4>(fv, safe, q);
        *reinterpret_cast<uint32_t*>(xq + frag_offset(t, j >> 1, j & 1, nb) + (f & 3) * 4) = pack_q4(q);
      }
    }
  } else {
    for (int j = threadIdx.x; j < hb; j += 256) {
      uint4 q = make_uint4(0u, 0u, 0u, 0u);
      if (t < T) {
        const float* p = row + j * 16;
        const float4 v4[4] = {ld4(p, 0), ld4(p, 1), ld4(p, 2), ld4(p, 3)};
        q = q8x16(v4, safe);
      }
      *reinterpret_cast<uint4*>(xq + frag_offset(t, j >> 1, j & 1, nb)) = q;
    }
  }
  if (threadIdx.x == 0) xd[t] = sc;
}

// ---------------------------------------------------------------- int8 GEMV (decode)
//
// A workgroup owns one H-row tile of the weight (for SwiGLU the gate and up tiles together): one
// contiguous chunk of the repacked layout. Every (row, block) item's product
//   q8: p = float(S_b) * xd_b        q4: p = float(S_b) * (ws_b * xd_b)
// goes to LDS (each multiply rounds exactly as on the CPU); then one lane per
// (token, row) folds its products in block order with plain adds and applies the epilogue.
// Consecutive lanes take consecutive items, so every weight load instruction reads one
// contiguous run. Every dispatch starts with cold instruction caches, so the kernels are kept
// short and issue all of their loads before any dependent work.

struct GemvLds {
  int8_t* q;  // [NT][kpad]
  float* d;   // [NT][nb]
  int* s;     // [NT][nb]
  float* p;   // [NSEL][NT][H][pst]
  int kpad, pst;
};

template <int NT>
__device__ __forceinline__ GemvLds gemv_lds(unsigned char* smem, int K, int nb) {
  GemvLds L;
  L.kpad = (K + 15) & ~15;
  L.pst = fold_stride(nb);
  L.q = reinterpret_cast<int8_t*>(smem);
  L.d = reinterpret_cast<float*>(smem + NT * L.kpad);
  L.s = reinterpret_cast<int*>(L.d + NT * nb);
  L.p = reinterpret_cast<float*>(smem + NT * L.kpad + ((NT * nb * 8 + 15) & ~15));
  return L;
}

// Fold lanes: one lane per row chain. Without SwiGLU lane c folds pair c = t * R + r (token t,
// row r). With SwiGLU every 16-lane row holds 8 pairs, gate chains in lanes 0-7 and the up chains
// of the same pairs in lanes 8-15, so one row_swap8 brings a row's up sum to its gate lane.
template <bool SW>
__device__ __forceinline__ void fold_lane(int tid, int& sel, int& pr) {
  sel = SW ? (tid >> 3) & 1 : 0;
  pr = SW ? ((tid >> 4) << 3) | (tid & 7) : tid;
}

// Threads the fold lanes of T tokens by R rows span.
template <bool SW>
__device__ __forceinline__ int fold_lanes(int T, int R) {
  return SW ? ((T * R + 7) >> 3) << 4 : T * R;
}

// Last phase of the small GEMV (and of the streaming GEMV without a fold wave): each fold lane
// sums its chain's row of products (the workgroup's R rows start at weight row n0, of which
// `rows` are real) and applies the epilogue. e_res and e_s come from chain_epilogue_operands.
// QOUT (SwiGLU, one token, R = 32, n0 a multiple of 32: the fold lanes are wave 0 and its gate
// lanes hold one 32-block of the output row): the block is also quantized as the activation
// quantizer does it (quantize_act_row, kernels_ref.cpp:23-37: the amax, s = amax / 127, each value's
// rounding that of its division, the block sum of q), for the next GEMV to take pre-quantized.
template <int WDT, int NT, bool SW, bool QOUT = false>
__device__ __forceinline__ void gemv_fold(const GemvArgs& a, const GemvLds& L, const GemvTarget& tg, int n0, int R,
                                          int rows, int tid, float e_res, float e_s) {
  static_assert(!QOUT || SW, "quantized output: SwiGLU only");
  if ((tid & ~63) >= fold_lanes<SW>(a.T, R)) return;  // whole waves only: the swap needs every lane
  int sel, pr;
  fold_lane<SW>(tid, sel, pr);
  // one token (NT == 1): every live lane has pr < R, so the division is skipped
  const int ft = NT == 1 ? 0 : pr / R, fr = pr - ft * R, fn = n0 + fr;
  const bool live = pr < a.T * R && fr < rows && fn < tg.N;
  float v = fold_chain(L.p + (live ? (sel * NT + ft) * R + fr : 0) * L.pst, a.nb);
  if (WDT == WQ8) v = v * e_s;
  if (SW) {
    const float up = row_swap8(v);
    const float hv = silu_exact(v) * up;
    const bool mine = live && sel == 0;
    if (mine) tg.y[(int64_t)ft * tg.N + fn] = hv;
    if (QOUT && a.oq) {  // uniform; every lane of wave 0 runs the reductions
      const float am = wave_max(mine ? fabsf(hv) : 0.f);
      const float d = am / 127.0f;
      int q;
      elm_q8_group<1>(&hv, d == 0.f ? 1.f : d, &q);
      const int sm = wave_sum_i(mine ? q : 0);
      if (mine) {
        a.oq[fn] = (int8_t)q;
        if (fr == 0) {
          a.od[fn / kBlock] = d;
          a.os[fn / kBlock] = sm;
        }
      }
    }
  } else if (live) {
    tg.y[(int64_t)ft * tg.N + fn] = tg.res ? v + e_res : v;
  }
}

// Epilogue operands of a fold lane (gemv_fold's mapping), loaded early: its chain's row scale
// (q8) and, without SwiGLU, the residual.
template <int WDT, bool SW>
__device__ __forceinline__ void chain_epilogue_operands(const GemvArgs& a, const GemvTarget& tg, int n0, int R, int rows,
                                                        int tid, float& e_res, float& e_s) {
  int sel, pr;
  fold_lane<SW>(tid, sel, pr);
  const int ft = pr / R, fr = pr - ft * R, fn = n0 + fr;
  const bool ok = tid < fold_lanes<SW>(a.T, R) && pr < a.T * R && fr < rows && fn < tg.N;
  // unconditional loads from clamped indices (a conditional load makes the compiler's earlier waits
  // cover it); lanes that fold nothing drop the values
  const int fc = min(fn, tg.N - 1), tc = min(ft, a.T - 1);
  e_s = WDT == WQ8 ? (sel ? a.tg[1].scales : tg.scales)[fc] : 1.f;
  e_res = !SW && tg.res ? tg.res[(int64_t)tc * tg.N + fc] : 0.f;
  if (!ok) {
    e_s = 1.f;
    e_res = 0.f;
  }
}

// Epilogue operands of a fold-wave lane, which folds both chains of pair `lane` (token
// lane / R, row lane % R), loaded early.
template <int WDT, bool SW>
__device__ __forceinline__ void pair_epilogue_operands(const GemvArgs& a, const GemvTarget& tg, int n0, int R, int rows,
                                                       int lane, float& e_res, float& e_s, float& e_su) {
  e_res = 0.f;
  e_s = e_su = 1.f;
  const int ft = lane / R, fr = lane - ft * R, fn = n0 + fr;
  if (lane < a.T * R && fr < rows && fn < tg.N) {
    if (WDT == WQ8) {
      e_s = tg.scales[fn];
      if (SW) e_su = a.tg[1].scales[fn];
    }
    if (!SW && tg.res) e_res = tg.res[(int64_t)ft * tg.N + fn];
  }
}

// A value pinned in scalar registers at this point: the compiler can no longer turn a select
// between such values back into a load through a selected address.
template <typename V>
__device__ __forceinline__ V pin_sgpr(V v) {
  asm volatile("" : "+s"(v));
  return v;
}

// A pinned pointer restated as global memory (the pin hides where it came from; without this the
// accesses through it become flat instructions, which also count against the LDS wait counter).
template <typename P>
__device__ __forceinline__ P* pin_global(P* p) {
  __attribute__((address_space(1))) P* g = (__attribute__((address_space(1))) P*)p;
  asm volatile("" : "+s"(g));
  return (P*)g;
}

// Target ti (uniform) read through the kernel-argument segment pointer: an indexed access to the
// by-value argument would make the compiler copy it to scratch memory. The kernel's only argument
// is the struct, so it sits at offset 0 of the segment.
__device__ __forceinline__ GemvTarget target_at(const GemvArgs& a, int ti) {
  (void)a;
  typedef const GemvArgs __attribute__((address_space(4)))* KernArgs;
  const KernArgs ka = (KernArgs)__builtin_amdgcn_kernarg_segment_ptr();
  GemvTarget t;
  t.data = pin_global(ka->tg[ti].data);
  t.scales = pin_global(ka->tg[ti].scales);
  t.y = pin_global(ka->tg[ti].y);
  t.res = pin_global(ka->tg[ti].res);
  t.N = ka->tg[ti].N;
  t.tiles = ka->tg[ti].tiles;
  return t;
}

// The target owning workgroup (or tile) index `wg`, which is made relative to that target. A launch
// of one target (MT false: every call but a fused QKV) reads the first target's fields with its other
// launch arguments in one batch of scalar loads; with more, the tile starts pick the target and its
// fields take one more (uniform) load.
template <bool SW, bool MT = true>
__device__ __forceinline__ GemvTarget gemv_target(const GemvArgs& a, int& wg) {
  if (SW || !MT) return a.tg[0];
  const int n = a.n_targets;
  const int ts1 = pin_sgpr(a.tile_start[1]), ts2 = pin_sgpr(a.tile_start[2]), ts3 = pin_sgpr(a.tile_start[3]);
  const int ti = (n > 1 && wg >= ts1) + (n > 2 && wg >= ts2) + (n > 3 && wg >= ts3);
  wg -= ti == 0 ? 0 : ti == 1 ? ts1 : ti == 2 ? ts2 : ts3;
  return target_at(a, ti);
}

// Small decode GEMV: x quantized inside the workgroup (4 values per thread, 8 threads per block,
// kSmallPass values per pass), at most two items per thread held in registers before the products
// (longer tiles loop). A workgroup takes up to kSmallMaxAct activation values (T * K).
constexpr int kSmallPass = kGemvThreads * 4;
constexpr int kSmallMaxAct = 4 * kSmallPass;

// NORM: x is the un-normalized row and the workgroup applies edgelm's RMSNORM to it first
// (cpu::rmsnorm, kernels_cpu.cpp:326-335, in the order of rmsnorm_kernel: squares grouped by
// dot_f32_scalar's four accumulators, four in-order sums, (s0 + s1) + (s2 + s3), then
// (x * inv) * w), so that RMSNORM and the matmul after it take one launch.
template <int WDT, int NT, bool SW, bool NORM, bool MT>
__global__ __launch_bounds__(kGemvThreads) void gemv_small_kernel(const GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int G = WDT == WQ8 ? 32 : 16;
  // every launch argument this kernel reads, in scalar registers before anything else: the
  // compiler issues their loads as one batch (one round trip to the argument segment) instead of
  // loading each near its first use, behind the waits for the ones before
  // MT (a fused QKV): every target's fields too, through one statement as outputs, so that the
  // target is picked by selects instead of a second batch of loads at its index (which the first
  // activation load would wait for)
  int ts1 = a.tile_start[1], ts2 = a.tile_start[2], ts3 = a.tile_start[3], ntg = a.n_targets;
  const uint8_t *d0 = a.tg[0].data, *d1 = a.tg[1].data, *d2 = a.tg[2].data, *d3 = a.tg[3].data;
  const float *s0 = a.tg[0].scales, *s1 = a.tg[1].scales, *s2 = a.tg[2].scales, *s3 = a.tg[3].scales;
  float *y0 = a.tg[0].y, *y1 = a.tg[1].y, *y2 = a.tg[2].y, *y3 = a.tg[3].y;
  const float *q0 = a.tg[0].res, *q1 = a.tg[1].res, *q2 = a.tg[2].res, *q3 = a.tg[3].res;
  int n0t = a.tg[0].N, n1t = a.tg[1].N, n2t = a.tg[2].N, n3t = a.tg[3].N;
  // (the RMSNORM operands go through the same statement: a second statement's loads would be a
  // second batch)
  if constexpr (MT && !SW) {
#define ELM_GS_MT_OUT                                                                                   \
  "+s"(ts1), "+s"(ts2), "+s"(ts3), "+s"(ntg), "+s"(d0), "+s"(d1), "+s"(d2), "+s"(d3), "+s"(s0), "+s"(s1), \
      "+s"(s2), "+s"(s3), "+s"(y0), "+s"(y1), "+s"(y2), "+s"(y3), "+s"(q0), "+s"(q1), "+s"(q2), "+s"(q3),  \
      "+s"(n0t), "+s"(n1t), "+s"(n2t), "+s"(n3t)
    if constexpr (NORM)
      asm volatile("" : ELM_GS_MT_OUT
                   : "s"(a.x), "s"(a.T), "s"(a.K), "s"(a.nb), "s"(a.H), "s"(a.rsub), "s"(a.nw), "s"(a.eps),
                     "s"(a.tile_start[4]));
    else
      asm volatile("" : ELM_GS_MT_OUT
                   : "s"(a.x), "s"(a.T), "s"(a.K), "s"(a.nb), "s"(a.H), "s"(a.rsub), "s"(a.tile_start[4]));
#undef ELM_GS_MT_OUT
  } else {
    asm volatile("" ::"s"(a.x), "s"(a.T), "s"(a.K), "s"(a.nb), "s"(a.H), "s"(a.rsub), "s"(a.tg[0].data),
                 "s"(a.tg[0].scales), "s"(a.tg[0].y), "s"(a.tg[0].res), "s"(a.tg[0].N));
    if (NORM) asm volatile("" ::"s"(a.nw), "s"(a.eps));
    if (SW) asm volatile("" ::"s"(a.tg[1].data), "s"(a.tg[1].scales));
  }
  const int K = a.K, nb = a.nb, T = a.T, H = a.H, tid = threadIdx.x;
  const GemvLds L = gemv_lds<NT>(smem, K, nb);
  // a workgroup takes RS rows (a power of two dividing H) of an H-row tile: part `part` of tile `tile`
  const int RS = a.rsub ? a.rsub : H, lgRS = __builtin_ctz(RS), lgsplit = __builtin_ctz(H) - lgRS;
  const int nel = T * K;
  // 1. every pass's activation values (first, before the target is picked: their wait does not
  // cover the weight loads issued next; loads past the end repeat the last float4), with NORM also
  // the norm weights
  const int e0 = tid * 4;
  constexpr int XP = kSmallMaxAct / kSmallPass;
  float4 xv[XP], nv[XP];
#pragma unroll
  for (int p = 0; p < XP; ++p) {
    const int e = min(p * kSmallPass + e0, nel - 4);
    xv[p] = *reinterpret_cast<const float4*>(a.x + e);  // unconditional: keeps the wait counts exact
    if (NORM) nv[p] = *reinterpret_cast<const float4*>(a.nw + (NT == 1 ? e : e - e / K * K));  // one token: e < K
  }
  __builtin_amdgcn_sched_barrier(0);  // the activation requests go out before the target selection
  int wg = blockIdx.x;
  GemvTarget tg;
  if constexpr (MT && !SW) {
    const int ti = (ntg > 1 && wg >= ts1) + (ntg > 2 && wg >= ts2) + (ntg > 3 && wg >= ts3);
    wg -= ti == 0 ? 0 : ti == 1 ? ts1 : ti == 2 ? ts2 : ts3;
    tg.data = pin_global(ti == 0 ? d0 : ti == 1 ? d1 : ti == 2 ? d2 : d3);
    tg.scales = pin_global(ti == 0 ? s0 : ti == 1 ? s1 : ti == 2 ? s2 : s3);
    tg.y = pin_global(ti == 0 ? y0 : ti == 1 ? y1 : ti == 2 ? y2 : y3);
    tg.res = pin_global(ti == 0 ? q0 : ti == 1 ? q1 : ti == 2 ? q2 : q3);
    tg.N = ti == 0 ? n0t : ti == 1 ? n1t : ti == 2 ? n2t : n3t;
    tg.tiles = 0;  // not read here
  } else {
    tg = gemv_target<SW, MT>(a, wg);
  }
  const int tile = wg >> lgsplit, part = wg & ((1 << lgsplit) - 1), n0 = tile * H + part * RS;
  const int64_t ibase = (int64_t)tile * H * nb + part * RS;  // item (row n0, block 0); (row n0 + r, block b) at + b H + r
  const uint8_t* const wd1 = SW ? a.tg[1].data : tg.data;
  const float* const ws1 = SW ? a.tg[1].scales : tg.scales;
  const int per_sel = RS * nb, items = (SW ? 2 : 1) * per_sel;

  // 2. weights of this thread's first two items
  v4u w[2][G / 16];
  float wsc[2] = {0.f, 0.f};
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    // unconditional (items past the last repeat it, unused): conditional loads would make the
    // compiler's waits for x cover these too
    const int it = min(u * kGemvThreads + tid, items - 1);
    const int sel = SW ? (it >= per_sel) : 0;
    const int j = it - sel * per_sel;
    const int64_t gi = ibase + (int64_t)(j >> lgRS) * H + (j & (RS - 1));
    const v4u* src = reinterpret_cast<const v4u*>((sel ? wd1 : tg.data) + gi * G);
    w[u][0] = src[0];
    if (G == 32) w[u][G / 16 - 1] = src[1];
    if (WDT == WQ4) wsc[u] = (sel ? ws1 : tg.scales)[gi];
  }
  // 3. epilogue operands of the folding lanes
  float e_res, e_s;
  chain_epilogue_operands<WDT, SW>(a, tg, n0, RS, RS, tid, e_res, e_s);
  if (NORM) {
    // 3b. RMSNORM of the T rows: squares to LDS as [t][accumulator][rowlen] (zero-padded: adding
    // +0.0 to a sum of squares changes nothing), lanes 4t .. 4t+3 sum row t's four accumulators,
    // inv_t = 1 / sqrt(ss / K + eps); then every value becomes (x * inv_t) * w
    const int K4 = K >> 2, rowlen = norm_rowlen(K);
    float* sq = L.p + (SW ? 2 : 1) * NT * RS * L.pst;
    float* inv_l = sq + NT * 4 * rowlen;
#pragma unroll
    for (int p = 0; p < XP; ++p) {
      const int e = p * kSmallPass + e0;
      if (e < nel) {
        const int t = NT == 1 ? 0 : e / K;  // one token: no division
        float* r = sq + t * 4 * rowlen + ((e - t * K) >> 2);
        r[0] = xv[p].x * xv[p].x;
        r[rowlen] = xv[p].y * xv[p].y;
        r[2 * rowlen] = xv[p].z * xv[p].z;
        r[3 * rowlen] = xv[p].w * xv[p].w;
      }
    }
    // +0.0 up to the next multiple of 16 terms
    for (int i = tid; i < T * 4 * 16; i += kGemvThreads)
      if (K4 + (i & 15) < ((K4 + 15) & ~15)) sq[(i >> 4) * rowlen + K4 + (i & 15)] = 0.f;
    lds_barrier();  // LDS only: the weight items stay in flight through the sums
    if (tid < 4 * T) {
      const float sacc = ordered_sum(sq + tid * rowlen, K4, 0.f);
      const float s01 = sacc + dpp_f<kDppQuadXor1>(sacc);
      const float ss = s01 + dpp_f<kDppQuadXor2>(s01);
      if ((tid & 3) == 0) inv_l[tid >> 2] = 1.0f / sqrtf(ss / (float)K + a.eps);
    }
    lds_barrier();
#pragma unroll
    for (int p = 0; p < XP; ++p) {
      const float inv = inv_l[NT == 1 ? 0 : min(p * kSmallPass + e0, nel - 4) / K];
      xv[p] = make_float4((xv[p].x * inv) * nv[p].x, (xv[p].y * inv) * nv[p].y, (xv[p].z * inv) * nv[p].z,
                          (xv[p].w * inv) * nv[p].w);
    }
  }
  // 4. quantize: block g = e0 / 32 spread over 8 consecutive lanes (4 values each)
  auto quantize = [&](int e, const float4 xx) {
    const float v[4] = {xx.x, xx.y, xx.z, xx.w};
    int qv[4], qs;
    const float sc = quant_block8x4(v, qv, qs);
    if (e < nel) {
      const int g = e >> 5, t = NT == 1 ? 0 : g / nb, b = g - t * nb;
      *reinterpret_cast<uint32_t*>(L.q + t * L.kpad + b * kBlock + (e & 31)) = pack_q4(qv);
      if ((e & 31) == 0) {
        L.d[t * nb + b] = sc;
        L.s[t * nb + b] = qs;
      }
    }
  };
#pragma unroll
  for (int p = 0; p < XP; ++p)
    if (p * kSmallPass < nel) quantize(p * kSmallPass + e0, xv[p]);
  __syncthreads();

  // 5. products
  for (int it = tid, u = 0; it < items; it += kGemvThreads, ++u) {
    const int sel = SW ? (it >= per_sel) : 0;
    const int j = it - sel * per_sel;
    v4u w0, w1;
    float ws;
    const int b = j >> lgRS, r = j & (RS - 1);
    if (u < 2) {
      w0 = u ? w[1][0] : w[0][0];
      w1 = u ? w[1][G / 16 - 1] : w[0][G / 16 - 1];
      ws = u ? wsc[1] : wsc[0];
    } else {
      const int64_t gi = ibase + (int64_t)b * H + r;
      const v4u* src = reinterpret_cast<const v4u*>((sel ? wd1 : tg.data) + gi * G);
      w0 = src[0];
      w1 = G == 32 ? src[1] : w0;
      ws = WDT == WQ4 ? (sel ? ws1 : tg.scales)[gi] : 0.f;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (t < T)
        L.p[((sel * NT + t) * RS + r) * L.pst + b] =
            item_product<WDT>(w0, w1, ws, L.q + t * L.kpad + b * kBlock, L.d[t * nb + b], L.s[t * nb + b]);
  }
  __syncthreads();
  gemv_fold<WDT, NT, SW>(a, L, tg, n0, RS, RS, tid, e_res, e_s);
}

// Streaming GEMV: T * K <= kStreamMaxAct activation bytes (staged in LDS).
constexpr int kStreamMaxAct = 16384;

// Adds row[b0 .. b1) to acc in block order. Up to 64 values (one batch of a row with 4-row
// tiles) are read before the first add, so the chain waits for LDS once; longer ranges repeat.
__device__ __forceinline__ float fold_range(float acc, const float* row, int b0, int b1) {
  int b = b0;
  for (; b < b1 && (b & 3); ++b) acc = acc + row[b];
  while (b + 4 <= b1) {
    const int ng = min((b1 - b) >> 2, 16);  // whole float4 groups this round
    float4 v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (i < ng) v[i] = *reinterpret_cast<const float4*>(row + b + 4 * i);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (i < ng) add4(acc, v[i]);
    b += 4 * ng;
  }
  for (; b < b1; ++b) acc = acc + row[b];
  return acc;
}

// Streaming decode GEMV for large weights: pre-quantized activation; a workgroup takes a.tpw
// consecutive H-row tiles (one contiguous chunk). NPW producer waves (P = 64 NPW threads)
// request the activation (copied straight into LDS) and then every weight item of the workgroup
// (at most IPT per thread), so nothing waits before the last request is out; vector loads retire
// in order, so the activation lands first. Item batch u (items u*P .. u*P+P-1: blocks u*P/H .. of
// each row) is multiplied as soon as it has landed and its products go to LDS. One more wave
// only folds: after batch u's barrier, one of its lanes per (token, row) adds the blocks of its
// row that the batch completed, in block order. The sequential fold (one dependent add per block,
// 448 per row at K = 14336) thus runs beside the products while later batches stream in, and
// only the last batch's share is left once the last weight has arrived. Without the fold wave
// (FW false: short rows, where the extra wave costs more than the chain) the producers fold at
// the end, one lane per (token, row).
template <int WDT, int NT, bool SW, int IPT, int NPW, int DEPTH, bool FW, bool QIN, bool QOUT, bool MT>
__global__ __launch_bounds__(64 * (NPW + FW)) void gemv_stream_kernel(const GemvArgs a) {
  static_assert(!QOUT || (SW && !FW && NT == 1), "quantized output: SwiGLU, one token, folds at the end");
  constexpr int P = 64 * NPW;  // producer threads
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int G = WDT == WQ8 ? 32 : 16;
  // every launch argument the kernel reads, in scalar registers first: one batch of loads, one
  // round trip to the argument segment (as the small GEMV)
  asm volatile("" ::"s"(a.T), "s"(a.K), "s"(a.nb), "s"(a.H), "s"(a.tpw));
  if (QIN)
    asm volatile("" ::"s"(a.x));
  else
    asm volatile("" ::"s"(a.xq), "s"(a.xd), "s"(a.xs));
  if (MT && !SW)
    asm volatile("" ::"s"(a.n_targets), "s"(a.tile_start[1]), "s"(a.tile_start[2]), "s"(a.tile_start[3]),
                 "s"(a.tile_start[4]));
  else
    asm volatile("" ::"s"(a.tg[0].data), "s"(a.tg[0].scales), "s"(a.tg[0].y), "s"(a.tg[0].res), "s"(a.tg[0].N),
                 "s"(a.tg[0].tiles));
  if (SW) asm volatile("" ::"s"(a.tg[1].data), "s"(a.tg[1].scales));
  if (QOUT) asm volatile("" ::"s"(a.oq), "s"(a.od), "s"(a.os));
  const int K = a.K, nb = a.nb, T = a.T, H = a.H, tid = threadIdx.x;
  const GemvLds L = gemv_lds<NT>(smem, K, nb);
  int wg = blockIdx.x;
  const GemvTarget tg = gemv_target<SW, MT>(a, wg);
  const int tile0 = wg * a.tpw;
  const int ntl = min(a.tpw, tg.tiles - tile0);
  const int R = a.tpw * H;      // LDS row slots per token
  const int rows = ntl * H;     // rows this workgroup owns
  const int per_tile = H * nb, per_sel = ntl * per_tile, items = (SW ? 2 : 1) * per_sel;
  const int lgH = __builtin_ctz(H), bpu = P >> lgH;
  const bool producer = tid < P;  // waves 0 .. NPW-1; wave NPW folds (FW)

  if (FW && !producer) {
    // fold wave: lane (ft, fr) owns row fr of token ft; gate (or the only weight) and up chains.
    // Batch u completes, for a row of local tile tl, blocks below (u + 1) P / H - tl nb (gate)
    // and below that minus ntl nb (up).
    // The chain is one dependent add per block: let this wave issue ahead of the producers
    // whenever it is ready, or it waits its turn behind their products on the same SIMD.
    __builtin_amdgcn_s_setprio(3);
    const int lane = tid - P;
    const int ft = NT == 1 ? 0 : lane / R, fr = lane - ft * R, ftl = fr >> lgH;
    const bool folder = lane < T * R && fr < rows;
    const float* const frow_g = L.p + (ft * R + fr) * L.pst;
    const float* const frow_u = L.p + ((NT + ft) * R + fr) * L.pst;
    float e_res, e_s, e_su;
    pair_epilogue_operands<WDT, SW>(a, tg, tile0 * H, R, rows, lane, e_res, e_s, e_su);
    float acc_g = 0.f, acc_u = 0.f;
    int done_g = 0, done_u = 0;
    __syncthreads();  // activation in LDS
    for (int u = 0; u < IPT; ++u) {
      __syncthreads();  // batch u's products in LDS
      if (folder) {
        const int lim = (u + 1) * bpu - ftl * nb;
        const int ng = min(max(lim, 0), nb);
        acc_g = fold_range(acc_g, frow_g, done_g, ng);
        done_g = ng;
        if (SW) {
          const int nu = min(max(lim - ntl * nb, 0), nb);
          acc_u = fold_range(acc_u, frow_u, done_u, nu);
          done_u = nu;
        }
      }
    }
    if (!folder) return;
    const int fn = tile0 * H + fr;
    if (fn >= tg.N) return;
    float out = WDT == WQ8 ? acc_g * e_s : acc_g;
    if (SW) {
      const float up = WDT == WQ8 ? acc_u * e_su : acc_u;
      out = silu_exact(out) * up;
    } else if (tg.res) {
      out = out + e_res;
    }
    tg.y[(int64_t)ft * tg.N + fn] = out;
    return;
  }

  const int64_t base = (int64_t)tile0 * per_tile;
  // A store the compiler cannot rule out (T is never negative): without one, loads from memory
  // that nothing in the kernel writes count as invariant and get sunk to their first use, which
  // would put them behind the waits below instead of all in flight at once.
  if (T < 0) tg.y[0] = 0.f;

  // 1. activation. QIN: the f32 values, four per producer thread per pass (eight 32-blocks per
  // wave), quantized below once they have landed. Otherwise the pre-quantized int8 values, block
  // scales and, for q4, block sums straight into LDS, where its rows are contiguous (K % 16 == 0):
  // wave w copies chunks w, w + NPW, ... of 1 KB (256 B).
  // QIN: 16 consecutive values per thread and pass (half a 32-block; the pair of lanes 2k, 2k + 1
  // holds one block), so each lane's share of the block's scale and reciprocal divisions covers 16
  // values (with 4 per lane, eight lanes per block, they were most of every workgroup's quantization
  // time)
  constexpr int QV = 16, QP = QIN ? kStreamQinPasses * 4 / QV : 1;
  float4 xv[QP][QV / 4];
  if (QIN) {
    const int nel = T * K;
#pragma unroll
    for (int p = 0; p < QP; ++p)
#pragma unroll
      for (int i = 0; i < QV / 4; ++i) {
        const float* px = a.x + min((p * P + tid) * QV + 4 * i, nel - 4);  // past the end: the last float4 again
        xv[p][i] = make_float4(px[0], px[1], px[2], px[3]);
      }
    __builtin_amdgcn_sched_barrier(0);  // these loads go out before the weight requests
  } else {
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int nq = T * K, nd = T * nb;
    for (int c = wave; c * 1024 < nq; c += NPW)
      if (c * 1024 + lane * 16 < nq) dma16(a.xq + c * 1024 + lane * 16, (unsigned char*)L.q + c * 1024);
    for (int c = wave; c * 64 < nd; c += NPW)
      if (c * 64 + lane < nd) {
        dma4(a.xd + c * 64 + lane, (unsigned char*)(L.d + c * 64));
        if (WDT == WQ4) dma4(a.xs + c * 64 + lane, (unsigned char*)(L.s + c * 64));
      }
  }
  if (!QIN) asm volatile("" ::: "memory");  // the weight requests below stay behind the activation's
  // 2. weight items of the first DEPTH batches in flight; batch u + DEPTH is requested once batch
  // u's products are out, so a wave whose requests stall (full memory queues) has already done
  // every product whose data has arrived. Requests past the last item repeat it.
  const uint8_t* const wd1 = SW ? a.tg[1].data : tg.data;
  const float* const ws1 = SW ? a.tg[1].scales : tg.scales;
  v4u w[IPT][G / 16];
  float wsc[IPT];
  auto request = [&](int u) {
    const int it = min(u * P + tid, items - 1);
    const int sel = SW ? (it >= per_sel) : 0;
    const int64_t gi = base + (it - sel * per_sel);
    const v4u* src = reinterpret_cast<const v4u*>((sel ? wd1 : tg.data) + gi * G);
    w[u][0] = __builtin_nontemporal_load(src);
    if (G == 32) w[u][G / 16 - 1] = __builtin_nontemporal_load(src + 1);
    wsc[u] = 0.f;
    if (WDT == WQ4) wsc[u] = __builtin_nontemporal_load((sel ? ws1 : tg.scales) + gi);
  };
  constexpr int D0 = DEPTH < IPT ? DEPTH : IPT;
#pragma unroll
  for (int u = 0; u < D0; ++u) request(u);
  asm volatile("" ::: "memory");  // these loads issued before anything waits
  // 3. the activation has landed once at most this wave's weight loads (two per item) are still
  // in flight (QIN: the compiler's wait for each pass's values, loaded first, leaves the weights in
  // flight); QIN quantizes it into LDS (edgelm's per-block rounding); the barrier makes every
  // wave's part visible
  if (QIN) {
    const int nel = T * K;
#pragma unroll
    for (int p = 0; p < QP; ++p) {
      if (p * P * QV < nel) {  // uniform; every lane runs the pass (the pair exchange below)
        const int e = (p * P + tid) * QV;
        float v[QV];
#pragma unroll
        for (int i = 0; i < QV / 4; ++i) {
          v[4 * i] = xv[p][i].x;
          v[4 * i + 1] = xv[p][i].y;
          v[4 * i + 2] = xv[p][i].z;
          v[4 * i + 3] = xv[p][i].w;
        }
        // quantize_act_row's block (kernels_ref.cpp:23-37): amax over both lanes, s = amax / 127,
        // every value's rounding that of its division (elm_q8_group), the block sum of q
        float am = 0.f;
#pragma unroll
        for (int i = 0; i < QV; ++i) am = fmaxf(am, fabsf(v[i]));
        am = fmaxf(am, dpp_f<kDppQuadXor1>(am));
        const float d = am / 127.0f;
        int q[QV];
        elm_q8_group<QV>(v, d == 0.f ? 1.f : d, q);
        int sm = 0;
#pragma unroll
        for (int i = 0; i < QV; ++i) sm += q[i];
        sm += dpp_i<kDppQuadXor1>(sm);
        if (e < nel) {  // nel is a multiple of 32: both lanes of a block, or neither
          const int g = e >> 5, t = NT == 1 ? 0 : g / nb, b = g - t * nb;  // one token: g < nb
          uint4 pk;
          pk.x = pack_q4({q[0], q[1], q[2], q[3]});
          pk.y = pack_q4({q[4], q[5], q[6], q[7]});
          pk.z = pack_q4({q[8], q[9], q[10], q[11]});
          pk.w = pack_q4({q[12], q[13], q[14], q[15]});
          *reinterpret_cast<uint4*>(L.q + t * L.kpad + b * kBlock + (e & 31)) = pk;
          if ((e & 31) == 0) {
            L.d[t * nb + b] = d;
            if (WDT == WQ4) L.s[t * nb + b] = sm;
          }
        }
      }
    }
  } else {
    wait_vm<2 * D0>();
  }
  __syncthreads();
  float e_res = 0.f, e_s = 1.f;
  if (!FW) chain_epilogue_operands<WDT, SW>(a, tg, tile0 * H, R, rows, tid, e_res, e_s);

  // 4. products into LDS in request order (each waits only for its own loads), one barrier per
  // batch. H is a power of two dividing P, so a thread's row within its tile never changes and
  // its block advances by P / H per batch; no integer division per item.
  const int r_in = tid & (H - 1), q0 = tid >> lgH;
  const float inv_nb = 1.0f / (float)nb;
  const int tstride = R * L.pst, sstride = NT * tstride, prow = r_in * L.pst;
#pragma unroll
  for (int u = 0; u < IPT; ++u) {  // every batch, also empty ones: straight-line code, exact waits
    {
      const int it = u * P + tid;
      if (it < items) {
        const int sel = SW ? (it >= per_sel) : 0;
        int b = u * bpu + q0 - (sel ? ntl * nb : 0);  // block position across this selection's tiles
        int off = prow + (sel ? sstride : 0);
        if (a.tpw > 1) {
          // tile = floor(b / nb): (b + 0.5) / nb is at least 0.5 / nb away from an integer, far
          // more than the float error at these sizes (b < 4096)
          const int st = (int)(((float)b + 0.5f) * inv_nb);
          b -= st * nb;
          off += st * H * L.pst;
        }
        off += b;
#pragma unroll
        for (int t = 0; t < NT; ++t)
          if (t < T)
            L.p[off + t * tstride] = item_product<WDT>(w[u][0], w[u][G / 16 - 1], wsc[u], L.q + t * L.kpad + b * kBlock,
                                                       L.d[t * nb + b], L.s[t * nb + b]);
      }
    }
    if (u + DEPTH < IPT) request(u + DEPTH);
    if (FW) __syncthreads();  // also waits for this wave's product writes
  }
  if (!FW) {
    // 5. one lane per row chain folds its row in block order and applies the epilogue
    __syncthreads();
    gemv_fold<WDT, NT, SW, QOUT>(a, L, tg, tile0 * H, R, rows, tid, e_res, e_s);
  }
}

// ---------------------------------------------------------------- int8 MFMA GEMM (prefill)
//
// Workgroup = 4 waves over a (64 MT)-token x 128-row output tile; each wave owns an (32 MT) x 64 part
// as MT x 2 v_mfma_i32_32x32x32_i8 tiles with A = tokens and B = weight rows (a lane owns one output
// row of each tile, so the stores run along the row). One MFMA spans exactly one 32-block along K,
// so in the block-scale modes each block's int32 sums come out whole and are rescaled in block
// order (edgelm's scalar order: multiply then add, or one fused multiply-add in FAST mode); in the
// per-token q8 mode the int32 sums accumulate across all of K and one rescale finishes.
//
// K streams through a ring of D LDS slots, one 32-block per slot, filled by global_load_lds
// (direct to LDS: no staging registers, so D - 1 blocks are in flight). Every wave issues the same
// P DMA instructions per slot, so "my part of block b has landed" is a fixed vmcnt((D - 2) * P);
// one barrier per block then makes every part visible and frees the slot computed one block
// earlier (the per-block mode at 64-token tiles: one wait and one barrier per group of six blocks). Issues past
// the last block repeat the last block, which keeps the count fixed.
// Workgroups are numbered so that each XCD (workgroup index mod 8) takes a contiguous range of
// (row tile, token tile) pairs, token tile fastest: an XCD's L2 keeps its own weight rows.
//
// WV = 8 (block-scale modes without SwiGLU, for grids of fewer than two workgroups per CU): eight
// waves, two per SIMD. Waves 0-3 keep the roles above, DMA included (the same P instructions per
// slot, the same wait counts); waves 4-7 issue no DMA. Each of the eight computes one of the two
// 32-row MFMA tiles that a wave of the four-wave form computes (wave w: tile w >> 2 of the part of
// wave w & 3), so a block's VALU rescale on one wave of a SIMD can run while the other wave of the
// SIMD waits on its MFMA or its LDS reads. Same arithmetic, same order, same bits.

static_assert(kGemmTileT == 128 && kGemmTileN == 128, "GEMM tile: the token padding covers both tile heights");

// Target ti (uniform) of a GEMM launch read through the kernel-argument segment pointer.
__device__ __forceinline__ GemmTarget gemm_target_at(int ti) {
  typedef const GemmArgs __attribute__((address_space(4)))* KernArgs;
  const KernArgs ka = (KernArgs)__builtin_amdgcn_kernarg_segment_ptr();
  GemmTarget t;
  t.data = pin_global(ka->tg[ti].data);
  t.scales = pin_global(ka->tg[ti].scales);
  t.y = pin_global(ka->tg[ti].y);
  t.res = pin_global(ka->tg[ti].res);
  t.N = ka->tg[ti].N;
  t.ntiles = ka->tg[ti].ntiles;
  return t;
}

template <int WDT, bool SW, bool TOK, int MT, int KBO>
struct GemmRing {
  static constexpr int TT = 64 * MT;
  static constexpr int NSEL = SW ? 2 : 1;
  static constexpr bool BLOCKX = !TOK;
  static constexpr int ACT = TT * 32;                                    // [TT/32 groups][2 halves][32][16]
  static constexpr int WSEL = WDT == WQ8 ? kGemmTileN * 32 : kGemmTileN * 20;  // q8 [2][128][16]; q4 [128][16] + [128] f32
  static constexpr int XD = BLOCKX ? TT * 4 : 0;
  static constexpr int SLOT = ACT + NSEL * WSEL + XD;
  // ring depth: whole block groups where blocks are grouped per barrier (KB below), one block otherwise
  static constexpr int KBQ = TOK && WDT == WQ8 && !SW && KBO == 0 ? (MT == 1 ? 4 : 2) : (KBO ? KBO : 1);
  static constexpr int D0 = (76 * 1024) / SLOT < 4 ? 4 : (76 * 1024) / SLOT;
  static constexpr int D = KBQ > 1 ? D0 / KBQ * KBQ : D0;
  static constexpr int P = 1 + NSEL + (BLOCKX ? 1 : 0);                        // DMA instructions per wave per slot
  // blocks per barrier: the per-token q8 loop is a few MFMAs per block, so its barrier, fragment
  // reads and DMA issues are grouped over KB blocks, and the ring holds whole groups
  static constexpr int KB = KBO ? KBO : TOK && WDT == WQ8 && !SW ? (MT == 1 ? 4 : 2) : 1;
  static_assert(D >= 2 * KB + 1 || (KB > 1 && D >= 3 * KB) || (BLOCKX && D >= 2 * KB), "ring too shallow for the block group");
  static constexpr int EP = SW ? 4 * 2 * 32 * 32 * 4 : 16;                     // SwiGLU epilogue: gate and up per wave
  static constexpr int BYTES = D * SLOT > EP ? D * SLOT : EP;
  static_assert((D - KB) * P < 64, "vmcnt range");
};

template <int WDT, bool SW, bool TOK, bool FAST, int MT, int KBO = 0, int WV = 4>
__global__ __launch_bounds__(64 * WV) __attribute__((amdgpu_waves_per_eu(SW && MT == 2 ? 1 : 2))) void gemm_a8_kernel(
    const GemmArgs a) {
  typedef GemmRing<WDT, SW, TOK, MT, KBO> R;
  constexpr int TT = R::TT, NSEL = R::NSEL, D = R::D;
  constexpr bool BLOCKX = R::BLOCKX;
  static_assert(WV == 4 || (WV == 8 && !SW && (R::KB == 1 || TOK || BLOCKX)), "eight waves: without SwiGLU");
  constexpr int NTW = WV == 8 ? 1 : 2;  // 32-row MFMA tiles per wave
  __shared__ __align__(16) unsigned char ring[R::BYTES];
  __shared__ __align__(16) float Lxdt[TOK ? TT : 4];

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
  // wave: 0 .. WV - 1; role: the four-wave form's wave whose part this wave shares (DMA by waves 0-3
  // only); nt0: the first of this wave's 32-row tiles within that part
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), role = wave & 3, wt = role >> 1, wr = role & 1;
  const int nt0 = WV == 8 ? wave >> 2 : 0;
  const bool dma_wave = WV == 4 || wave < 4;
  const int nb = a.nb, H = a.H;
  // workgroup -> (row tile, token tile)
  const int n = pin_sgpr(a.n_targets);
  const int ts1 = pin_sgpr(a.tile_start[1]), ts2 = pin_sgpr(a.tile_start[2]), ts3 = pin_sgpr(a.tile_start[3]);
  const int ts4 = pin_sgpr(a.tile_start[4]);
  const int rtn = SW ? a.tg[0].ntiles : n == 1 ? ts1 : n == 2 ? ts2 : n == 3 ? ts3 : ts4;  // row tiles in all
  const int ntt = (a.T + TT - 1) / TT;  // token tiles: each starts below T
  const int total = rtn * ntt, chunk = (total + 7) >> 3;
  const int id = (int)(blockIdx.x & 7) * chunk + (int)(blockIdx.x >> 3);
  if (id >= total) return;
  int rt = id / ntt;
  const int tt = id - rt * ntt;
  const int ti = SW ? 0 : (n > 1 && rt >= ts1) + (n > 2 && rt >= ts2) + (n > 3 && rt >= ts3);
  rt -= ti == 0 ? 0 : ti == 1 ? ts1 : ti == 2 ? ts2 : ts3;
  const GemmTarget tg = SW ? a.tg[0] : gemm_target_at(ti);
  const int r0 = rt * kGemmTileN, t0 = tt * TT;
  const int rows_pad = (tg.N + kPadRows - 1) / kPadRows * kPadRows;  // the weight's padded rows
  auto wdata = [&](int s) { return SW && s ? a.tg[1].data : tg.data; };
  auto wscal = [&](int s) { return SW && s ? a.tg[1].scales : tg.scales; };

  // DMA roles. Activation: 1 KB fragment (group, block) = [half][32 tokens][16 B], the same layout
  // in HBM and in the slot; wave w copies group w (MT = 2) or half w & 1 of group w >> 1 (MT = 1,
  // lanes 0-31). q8 weights: the slot holds 16-byte position p = 2 r + (h ^ bit 3 of r) for half h
  // of row r, so that wave w's lanes read rows 32 w .. 32 w + 31 as consecutive 16-byte chunks of
  // the repacked layout, and 16 lanes reading one half of 16 rows touch every LDS bank once.
  // q4 weights: lane row (w & 1) * 64 + lane, data (w < 2) or scale.
  const int drow = WDT == WQ8 ? role * 32 + (lane >> 1) : (role & 1) * 64 + lane;
  const int dhalf = (lane & 1) ^ ((drow >> 3) & 1);  // q8: the half that lane fills
  const int wrow = min(r0 + drow, rows_pad - 1);
  const int64_t rbase = (int64_t)(wrow / H) * nb * H + (wrow % H);  // item of (wrow, block 0)
  // this lane's byte offsets at block 0 (the host keeps both arrays below 2 GB); a block adds a
  // uniform stride to the scalar base: 1 KB of activation, H items of weight, Tpad scales
  const uint32_t xoff = (uint32_t)(((int64_t)((t0 >> 5) + (MT == 2 ? role : role >> 1)) * nb * 1024) +
                                   (MT == 2 ? lane * 16 : (role & 1) * 512 + l32 * 16));
  const uint32_t woff = (uint32_t)(WDT == WQ8 ? rbase * 32 + dhalf * 16 : rbase * 16);
  const uint32_t soff = (uint32_t)(rbase * 4);
  const uint32_t doff = (uint32_t)((t0 + role * (TT / 4) + lane) * 4);
  constexpr uint32_t G = WDT == WQ8 ? 32 : 16;
  const uint32_t wstride = (uint32_t)H * G, sstride = (uint32_t)H * 4, dstride = (uint32_t)a.Tpad * 4;
  const unsigned ring_lds = (unsigned)(size_t)(LdsBytes)ring;
  auto issue = [&](int blk, int slot) {
    if (!dma_wave) return;  // uniform per wave: waves 4-7 of the eight-wave form copy nothing
    const uint32_t ub = (uint32_t)min(blk, nb - 1);
    const unsigned sb = ring_lds + (unsigned)slot * R::SLOT;
    if (MT == 2 || lane < 32) dma16s(a.xq + ub * 1024u, xoff, sb + role * (MT == 2 ? 1024 : 512));
#pragma unroll
    for (int sl = 0; sl < NSEL; ++sl) {
      const unsigned wb = sb + R::ACT + sl * R::WSEL;
      if (WDT == WQ8 || role < 2) {
        dma16s(wdata(sl) + ub * wstride, woff, wb + role * 1024);
      } else {
        dma4s((const unsigned char*)wscal(sl) + ub * sstride, soff, wb + 2048 + (role - 2) * 256);
      }
    }
    if (BLOCKX && lane < TT / 4)
      dma4s((const unsigned char*)a.xd + ub * dstride, doff, sb + R::ACT + NSEL * R::WSEL + role * TT);
  };

  v16i iacc[NSEL][MT][NTW];
  float facc[NSEL][MT][NTW][16];
#pragma unroll
  for (int s = 0; s < NSEL; ++s)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          iacc[s][mt][nt][i] = 0;
          facc[s][mt][nt][i] = 0.f;
        }
  v16i zero;
#pragma unroll
  for (int i = 0; i < 16; ++i) zero[i] = 0;

  // one 32-block from a slot: MT x NTW MFMAs per wave (per weight selection)
  auto block = [&](int slot) {
    const unsigned char* sb = ring + slot * R::SLOT;
    v4i A[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) A[mt] = *reinterpret_cast<const v4i*>(sb + ((wt * MT + mt) * 64 + lane) * 16);
#pragma unroll
    for (int s = 0; s < NSEL; ++s) {
      const unsigned char* wb = sb + R::ACT + s * R::WSEL;
      v4i B[NTW];
      float c[NTW];
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) {
        const int rl = wr * 64 + (nt0 + nt) * 32 + l32;
        c[nt] = 1.f;
        if (WDT == WQ8) {
          B[nt] = *reinterpret_cast<const v4i*>(wb + (2 * rl + (h ^ ((rl >> 3) & 1))) * 16);
        } else {
          B[nt] = q4_operand16(*reinterpret_cast<const uint4*>(wb + rl * 16), h);
          c[nt] = reinterpret_cast<const float*>(wb + 2048)[rl];
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float xv[16];
        if (BLOCKX) {
          const float* xs = reinterpret_cast<const float*>(sb + R::ACT + NSEL * R::WSEL);
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const float4 x4 = *reinterpret_cast<const float4*>(&xs[wt * 32 * MT + mt * 32 + 8 * g + 4 * h]);
            xv[4 * g] = x4.x;
            xv[4 * g + 1] = x4.y;
            xv[4 * g + 2] = x4.z;
            xv[4 * g + 3] = x4.w;
          }
        }
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
          if (TOK && WDT == WQ8) {
            iacc[s][mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[mt], B[nt], iacc[s][mt][nt], 0, 0, 0);
          } else {
            const v16i S = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[mt], B[nt], zero, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              // q8: p = float(S) * xd; q4 (S = 16 * S_b, c = ws): p = float(S) * (c * xd) = 16 * edgelm's product
              // (c * xd rounds as on the CPU; 16 times a product or a sum of multiples of 2^-149 is exact, so
              // the q4 fold stays 16 times edgelm's, subnormal range included, up to 2^124 in magnitude, and
              // one multiply by 1/16 before the store restores it)
              const float m = WDT == WQ8 ? xv[i] : BLOCKX ? c[nt] * xv[i] : c[nt];
              if (FAST) {
                facc[s][mt][nt][i] = __builtin_fmaf((float)S[i], m, facc[s][mt][nt][i]);
              } else {
                facc[s][mt][nt][i] = facc[s][mt][nt][i] + (float)S[i] * m;
              }
            }
          }
        }
      }
    }
  };

  // per-token scales of the tile's tokens (the per-token mode's epilogue reads them from LDS)
  if (TOK && tid < TT) Lxdt[tid] = a.xd[t0 + tid];
  if constexpr (WV == 8 && WDT == WQ4 && BLOCKX && R::KB == 1) {
    // Eight waves, q4, edgelm's per-block rescale, pipelined by one block (block j in slot j % D): step b
    // starts block b's MFMAs from operands read in step b - 1, reads block b's token scales from its
    // slot, then block b + 1's operands, and rescales while those reads are in flight. Slot (b - 1) % D
    // is refilled with block b + D - 1 after the barrier at the top of step b, when no wave reads it
    // any more; block b + 1 has landed once at most D - 3 blocks are in flight. Measured at T = 512
    // against the loop below: q4 4096 x 4096 60.4 -> 57.8 us, 4096 x 14336 174.0 -> 162.4 us; q8 lost
    // (48.0 -> 51.7, 127.4 -> 146.4 us), and prefetching the 16 token scales as well spilled or lost.
    // (128-token tiles, and 64-token tiles with ELMH_GEMM_KB=1: the grouped loop below measured faster.)
    static_assert(D >= 4, "ring too shallow for the eight-wave pipeline");
    auto read_ops = [&](v4i (&A)[MT], v4i& B, float& c, int blk) {
      const unsigned char* sb = ring + (blk % D) * R::SLOT;
      const unsigned char* wb = sb + R::ACT;
      const int rl = wr * 64 + nt0 * 32 + l32;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) A[mt] = *reinterpret_cast<const v4i*>(sb + ((wt * MT + mt) * 64 + lane) * 16);
      c = 1.f;
      if (WDT == WQ8) {
        B = *reinterpret_cast<const v4i*>(wb + (2 * rl + (h ^ ((rl >> 3) & 1))) * 16);
      } else {
        B = q4_operand16(*reinterpret_cast<const uint4*>(wb + rl * 16), h);
        c = reinterpret_cast<const float*>(wb + 2048)[rl];
      }
    };
    auto step = [&](v4i (&A)[MT], v4i& B, float& c, v4i (&A2)[MT], v4i& B2, float& c2, int b) {
      wait_vm<(D - 3) * R::P>();  // block b + 1 has landed (this wave's part)
      lds_barrier();              // every wave's part; every wave is done with block b - 1
      issue(b + D - 1, (b + D - 1) % D);
      v16i S[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) S[mt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[mt], B, zero, 0, 0, 0);
      const float* xs = reinterpret_cast<const float*>(ring + (b % D) * R::SLOT + R::ACT + R::WSEL);
      float4 x4[MT][4];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int g = 0; g < 4; ++g) x4[mt][g] = *reinterpret_cast<const float4*>(&xs[wt * 32 * MT + mt * 32 + 8 * g + 4 * h]);
      read_ops(A2, B2, c2, b + 1);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float4 v = x4[mt][i >> 2];
          const float xd = (i & 3) == 0 ? v.x : (i & 3) == 1 ? v.y : (i & 3) == 2 ? v.z : v.w;
          // as block(): q8 p = float(S) * xd; q4 p = float(S) * (c * xd), 16 times edgelm's product
          const float m = WDT == WQ8 ? xd : c * xd;
          if (FAST) {
            facc[0][mt][0][i] = __builtin_fmaf((float)S[mt][i], m, facc[0][mt][0][i]);
          } else {
            facc[0][mt][0][i] = facc[0][mt][0][i] + (float)S[mt][i] * m;
          }
        }
    };
#pragma unroll
    for (int i = 0; i < D - 1; ++i) issue(i, i);
    wait_vm<(D - 2) * R::P>();  // block 0 has landed
    lds_barrier();
    v4i A0[MT], B0, A1[MT], B1;
    float c0, c1;
    read_ops(A0, B0, c0, 0);
    int b = 0;
    for (; b + 1 < nb; b += 2) {
      step(A0, B0, c0, A1, B1, c1, b);
      step(A1, B1, c1, A0, B0, c0, b + 1);
    }
    if (b < nb) step(A0, B0, c0, A1, B1, c1, b);  // reads block nb's slot (a repeat of the last block)
  } else if constexpr (BLOCKX && R::KB > 1) {
    // edgelm's per-block rescale with one wait and one barrier per group of KB blocks (block j in
    // slot j % D, D a multiple of KB) instead of per block. Step g waits until group g has landed,
    // refills group g - 1's slots (every wave is past them once the barrier opens) with the blocks
    // D - KB further on, then computes group g's blocks in order; the waves may drift by up to a
    // group between barriers. Blocks past the last are issued (repeats of it) but not computed.
    constexpr int KB = R::KB;
    static_assert(D % KB == 0 && D >= 2 * KB, "the ring holds whole groups, two at least");
    // Within a group the blocks are software-pipelined: block k + 2's operands are read from LDS
    // and block k + 1's MFMAs issued before block k's rescale, so reads and MFMAs run under it.
    struct Ops {
      v4i A[MT];
      v4i B[NTW];
      float c[NTW];
      float xv[MT][16];
    };
    auto read_ops = [&](Ops& o, int slot) {
      const unsigned char* sb = ring + slot * R::SLOT;
      const unsigned char* wb = sb + R::ACT;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) o.A[mt] = *reinterpret_cast<const v4i*>(sb + ((wt * MT + mt) * 64 + lane) * 16);
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) {
        const int rl = wr * 64 + (nt0 + nt) * 32 + l32;
        o.c[nt] = 1.f;
        if (WDT == WQ8) {
          o.B[nt] = *reinterpret_cast<const v4i*>(wb + (2 * rl + (h ^ ((rl >> 3) & 1))) * 16);
        } else {
          o.B[nt] = q4_operand16(*reinterpret_cast<const uint4*>(wb + rl * 16), h);
          o.c[nt] = reinterpret_cast<const float*>(wb + 2048)[rl];
        }
      }
      const float* xs = reinterpret_cast<const float*>(sb + R::ACT + NSEL * R::WSEL);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 x4 = *reinterpret_cast<const float4*>(&xs[wt * 32 * MT + mt * 32 + 8 * g + 4 * h]);
          o.xv[mt][4 * g] = x4.x;
          o.xv[mt][4 * g + 1] = x4.y;
          o.xv[mt][4 * g + 2] = x4.z;
          o.xv[mt][4 * g + 3] = x4.w;
        }
    };
    // block()'s arithmetic on operands already read: the MFMAs, then the rescale (skipped for the
    // repeats past the last block)
    auto mfma = [&](const Ops& o, v16i (&S)[MT][NTW]) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) S[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.A[mt], o.B[nt], zero, 0, 0, 0);
    };
    auto rescale = [&](const Ops& o, const v16i (&S)[MT][NTW]) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float m = WDT == WQ8 ? o.xv[mt][i] : o.c[nt] * o.xv[mt][i];
            if (FAST) {
              facc[0][mt][nt][i] = __builtin_fmaf((float)S[mt][nt][i], m, facc[0][mt][nt][i]);
            } else {
              facc[0][mt][nt][i] = facc[0][mt][nt][i] + (float)S[mt][nt][i] * m;
            }
          }
    };
#pragma unroll
    for (int i = 0; i < D - KB; ++i) issue(i, i);
    for (int b = 0; b < nb; b += KB) {
      wait_vm<(D - 2 * KB) * R::P>();  // group b / KB has landed (this wave's part)
      lds_barrier();                   // every wave's part; every wave is done with the group before
#pragma unroll
      for (int k = 0; k < KB; ++k) issue(b + D - KB + k, (b + D - KB + k) % D);
      const int s0 = b % D;  // the group's first slot (groups never wrap: D is a multiple of KB)
      // step k: read block k + 2's operands, start block k + 1's MFMAs, rescale block k
      Ops o[3];
      v16i S[2][MT][NTW];
      read_ops(o[0], s0);
      read_ops(o[1], s0 + 1);
      mfma(o[0], S[0]);
#pragma unroll
      for (int k = 0; k < KB; ++k) {
        if (k + 2 < KB) read_ops(o[(k + 2) % 3], s0 + k + 2);
        if (k + 1 < KB) mfma(o[(k + 1) % 3], S[(k + 1) & 1]);
        if (b + k < nb) rescale(o[k % 3], S[k & 1]);
      }
    }
  } else if constexpr (R::KB == 1) {
#pragma unroll
    for (int i = 0; i < D - 1; ++i) issue(i, i);
    int cs = 0, is = D - 1;  // slot to compute, slot to fill
    for (int b = 0; b < nb; ++b) {
      wait_vm<(D - 2) * R::P>();  // this wave's part of block b has landed
      lds_barrier();              // every wave's part has; every wave is done with block b - 1
      issue(b + D - 1, is);
      block(cs);
      cs = cs + 1 == D ? 0 : cs + 1;
      is = is + 1 == D ? 0 : is + 1;
    }
  } else {
    // per-token q8, software-pipelined over groups of KB blocks (block j in slot j % D; D is a
    // multiple of KB). Step g multiplies group g from registers while it reads group g + 1's
    // fragments and refills group g's slots with group g + D / KB, interleaved so that the DMA
    // issue, the LDS reads and the MFMAs of one wave overlap. Group g was read into registers in
    // step g - 1, before the barrier at the top of step g, so its slots are free; group g + 1 has
    // landed once at most D - 2 KB blocks are in flight. Blocks past the last (their slots repeat it)
    // are read but add zero.
    constexpr int KB = R::KB;
    static_assert(D % KB == 0, "the ring holds whole groups");
    auto read_group = [&](v4i (&A)[KB][MT], v4i (&B)[KB][NTW], int blk0, int k) {
      const unsigned char* sb = ring + ((blk0 % D) + k) * R::SLOT;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) A[k][mt] = *reinterpret_cast<const v4i*>(sb + ((wt * MT + mt) * 64 + lane) * 16);
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) {
        const int rl = wr * 64 + (nt0 + nt) * 32 + l32;
        B[k][nt] = *reinterpret_cast<const v4i*>(sb + R::ACT + (2 * rl + (h ^ ((rl >> 3) & 1))) * 16);
      }
    };
    auto step = [&](v4i (&A)[KB][MT], v4i (&B)[KB][NTW], v4i (&A2)[KB][MT], v4i (&B2)[KB][NTW], int b) {
      wait_vm<(D - 2 * KB) * R::P>();  // group b + KB has landed (this wave's part)
      lds_barrier();                   // every wave's part; every wave holds group b in registers
      const bool full = b + KB <= nb;  // uniform
#pragma unroll
      for (int k = 0; k < KB; ++k) {
        const bool ok = full || b + k < nb;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const v4i a4 = ok ? A[k][mt] : v4i{0, 0, 0, 0};
#pragma unroll
          for (int nt = 0; nt < NTW; ++nt)
            iacc[0][mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a4, B[k][nt], iacc[0][mt][nt], 0, 0, 0);
        }
        read_group(A2, B2, b + KB, k);
        issue(b + D + k, (b % D) + k);
        __builtin_amdgcn_sched_barrier(0);  // keep the MFMAs, reads and DMA of block k together
      }
    };
#pragma unroll
    for (int i = 0; i < D; ++i) issue(i, i);
    wait_vm<(D - KB) * R::P>();  // group 0 has landed
    lds_barrier();
    v4i A0[KB][MT], B0[KB][NTW], A1[KB][MT], B1[KB][NTW];
#pragma unroll
    for (int k = 0; k < KB; ++k) read_group(A0, B0, 0, k);
    int b = 0;
    for (; b + KB < nb; b += 2 * KB) {
      step(A0, B0, A1, B1, b);
      step(A1, B1, A0, B0, b + KB);
    }
    if (b < nb) step(A0, B0, A1, B1, b);
  }
  wait_vm<0>();  // the repeated last-block issues have landed before the ring is reused or freed
  lds_barrier();

  // epilogue: row r (lane), tokens t (accumulator index). Stores and residual loads go through
  // buffer resources that span the tile's valid tokens, and an offset past the end stands for a
  // row past N: the hardware drops such stores and returns 0 for such loads, so no lane branches.
  const int tv = min(TT, a.T - t0);  // valid tokens of the tile
  const uint32_t tbytes = (uint32_t)tv * (uint32_t)tg.N * 4u;
  const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(tg.y + (int64_t)t0 * tg.N, (short)0, (int)tbytes, 0x00020000);
  const bool has_res = !SW && tg.res != nullptr;
  const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(has_res ? tg.res + (int64_t)t0 * tg.N : tg.y), (short)0, has_res ? (int)tbytes : 0, 0x00020000);
  auto xd_tok = [&](float (&xt)[16], int mt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 x4 = *reinterpret_cast<const float4*>(&Lxdt[wt * 32 * MT + mt * 32 + 8 * g + 4 * h]);
      xt[4 * g] = x4.x;
      xt[4 * g + 1] = x4.y;
      xt[4 * g + 2] = x4.z;
      xt[4 * g + 3] = x4.w;
    }
  };
  if constexpr (SW) {
    // gate and up of each 32x32 tile go through this wave's LDS slice, so that silu (an expf)
    // is emitted once in a loop rather than once per accumulator
    float* const ep = reinterpret_cast<float*>(ring) + wave * (2 * 32 * 32);
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
      const int r = r0 + wr * 64 + (nt0 + nt) * 32 + l32;
      const int rc = min(r, tg.N - 1);
      const float ws = WDT == WQ8 ? tg.scales[rc] : 1.f;
      const float wsu = WDT == WQ8 ? a.tg[1].scales[rc] : 1.f;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float xt[16];
        if (TOK) xd_tok(xt, mt);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float g, u;
          if (WDT == WQ8) {
            g = TOK ? ((float)iacc[0][mt][nt][i] * xt[i]) * ws : facc[0][mt][nt][i] * ws;
            u = TOK ? ((float)iacc[NSEL - 1][mt][nt][i] * xt[i]) * wsu : facc[NSEL - 1][mt][nt][i] * wsu;
          } else {
            g = TOK ? (facc[0][mt][nt][i] * 0.0625f) * xt[i] : facc[0][mt][nt][i] * 0.0625f;
            u = TOK ? (facc[NSEL - 1][mt][nt][i] * 0.0625f) * xt[i] : facc[NSEL - 1][mt][nt][i] * 0.0625f;
          }
          ep[i * 64 + lane] = g;
          ep[1024 + i * 64 + lane] = u;
        }
        __builtin_amdgcn_wave_barrier();
        const int tb = wt * 32 * MT + mt * 32 + 4 * h;  // token within the tile
#pragma unroll 1
        for (int i = 0; i < 16; ++i) {
          const int t = tb + 8 * (i >> 2) + (i & 3);
          const float out = silu_exact(ep[i * 64 + lane]) * ep[1024 + i * 64 + lane];
          const int off = r < tg.N ? (t * tg.N + r) * 4 : 0x7FFFFFF0;
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, out), ry, off, 0, 0);
        }
        __builtin_amdgcn_wave_barrier();
      }
    }
    return;
  }
  // the residual choice is uniform: two branch-free copies of the store loop
  auto store_tiles = [&](auto res_tag) {
    constexpr bool RES = decltype(res_tag)::value;
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
      const int r = r0 + wr * 64 + (nt0 + nt) * 32 + l32;
      const int rc = min(r, tg.N - 1);
      const float ws = WDT == WQ8 ? tg.scales[rc] : 1.f;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float xt[16];
        if (TOK) xd_tok(xt, mt);
        const int tb = wt * 32 * MT + mt * 32 + 4 * h;
        float res[16];
        if (RES) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int t = tb + 8 * (i >> 2) + (i & 3);
            const int off = r < tg.N ? (t * tg.N + r) * 4 : 0x7FFFFFF0;
            res[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, off, 0, 0));
          }
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int t = tb + 8 * (i >> 2) + (i & 3);
          const int off = r < tg.N ? (t * tg.N + r) * 4 : 0x7FFFFFF0;
          float out;
          if (WDT == WQ8) {
            out = TOK ? ((float)iacc[0][mt][nt][i] * xt[i]) * ws : facc[0][mt][nt][i] * ws;
          } else {
            out = TOK ? (facc[0][mt][nt][i] * 0.0625f) * xt[i] : facc[0][mt][nt][i] * 0.0625f;
          }
          if (RES) out = out + res[i];
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, out), ry, off, 0, 0);
        }
      }
    }
  };
  if (has_res)
    store_tiles(std::true_type{});
  else
    store_tiles(std::false_type{});
}

// ---------------------------------------------------------------- int8 MFMA GEMM, small problems
//
// For GEMMs too small to give the LDS-ring kernel enough workgroups (SmolLM2-sized prefill: 576 to
// 1536 rows at T = 128 are 5 to 24 ring workgroups on 256 CUs), every wave owns one 32-token x
// 32-row output tile on its own: 4 independent waves per workgroup, no LDS ring and no barriers.
// Each lane loads its MFMA operands straight into registers (the activation fragment's 16 bytes,
// its weight row's 16 bytes of the block, the block scales), kWaveDepth blocks ahead, and the
// per-block int32 sums are rescaled in block order exactly as in the ring kernel, so both give
// the same bits. Waves sharing a token group or a row group share their operands through L2.
constexpr int kWaveDepth = 4;
constexpr int kWaveTile = 32;

template <int WDT, bool SW, bool TOK>
struct WaveOps {
  static constexpr int NSEL = SW ? 2 : 1;
  static constexpr bool BLOCKX = !TOK;
  v4i A;
  v4i B[NSEL];
  float c[NSEL];                // q4: ws of the lane's row and block
  float xv[BLOCKX ? 16 : 1];    // block scales of the lane's 16 tokens
};

template <int WDT, bool SW, bool TOK, bool FAST, int DEPTH = kWaveDepth>
__global__ __launch_bounds__(256) void gemm_wave_kernel(const GemmArgs a) {
  typedef WaveOps<WDT, SW, TOK> Ops;
  constexpr int NSEL = Ops::NSEL;
  constexpr bool BLOCKX = Ops::BLOCKX;
  __shared__ __align__(16) float ep_all[SW ? 4 * 2 * 32 * 32 : 4];
  __shared__ float xdt_all[TOK ? 4 * 32 : 4];
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int nb = a.nb, H = a.H;
  const int ngroups = (a.T + kWaveTile - 1) / kWaveTile;
  // wave -> (target, 32-row tile, token group), token group fastest
  int rt = (int)blockIdx.x * 4 + wave;
  const int g = rt % ngroups;
  rt /= ngroups;
  int ti = 0;
  const int n = SW ? 1 : a.n_targets;
  for (; ti < n; ++ti) {
    const int c = (a.tg[ti].N + kWaveTile - 1) / kWaveTile;
    if (rt < c) break;
    rt -= c;
  }
  if (ti >= n) return;  // past the last tile (uniform per wave; no barrier below)
  const GemmTarget tg = SW ? a.tg[0] : gemm_target_at(ti);
  const int r0 = rt * kWaveTile, t0 = g * kWaveTile;
  const int rows_pad = (tg.N + kPadRows - 1) / kPadRows * kPadRows;
  const int wrow = min(r0 + l32, rows_pad - 1);
  const int64_t rbase = (int64_t)(wrow / H) * nb * H + (wrow % H);  // item of (wrow, block 0)
  const uint8_t* const wd[2] = {tg.data, SW ? a.tg[1].data : tg.data};
  const float* const wsc[2] = {tg.scales, SW ? a.tg[1].scales : tg.scales};
  const int8_t* const xg = a.xq + (int64_t)g * nb * 1024 + lane * 16;

  auto load = [&](int blk, Ops& o) {
    blk = min(blk, nb - 1);
    o.A = *reinterpret_cast<const v4i*>(xg + (int64_t)blk * 1024);
    const int64_t it = rbase + (int64_t)blk * H;
#pragma unroll
    for (int s = 0; s < NSEL; ++s) {
      if (WDT == WQ8) {
        o.B[s] = *reinterpret_cast<const v4i*>(wd[s] + it * 32 + h * 16);
        o.c[s] = 1.f;
      } else {
        o.B[s] = q4_operand16(*reinterpret_cast<const uint4*>(wd[s] + it * 16), h);
        o.c[s] = wsc[s][it];
      }
    }
    if (BLOCKX) {
      const float* xs = a.xd + (int64_t)blk * a.Tpad + t0 + 4 * h;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 x4 = *reinterpret_cast<const float4*>(xs + 8 * q);
        o.xv[4 * q] = x4.x;
        o.xv[4 * q + 1] = x4.y;
        o.xv[4 * q + 2] = x4.z;
        o.xv[4 * q + 3] = x4.w;
      }
    }
  };

  v16i iacc[NSEL];
  float facc[NSEL][16];
  v16i zero;
#pragma unroll
  for (int i = 0; i < 16; ++i) zero[i] = 0;
#pragma unroll
  for (int s = 0; s < NSEL; ++s) {
    iacc[s] = zero;
#pragma unroll
    for (int i = 0; i < 16; ++i) facc[s][i] = 0.f;
  }
  // the int32 sums of a block; the rescale then folds them in block order
  auto sums = [&](const Ops& o, v16i (&S)[NSEL]) {
#pragma unroll
    for (int s = 0; s < NSEL; ++s) S[s] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.A, o.B[s], zero, 0, 0, 0);
  };
  auto rescale = [&](const Ops& o, const v16i (&S)[NSEL]) {
#pragma unroll
    for (int s = 0; s < NSEL; ++s)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        // q8: p = float(S) * xd; q4 (S = 16 * S_b, c = ws): p = float(S) * (c * xd) = 16 * edgelm's product
        const float m = WDT == WQ8 ? o.xv[BLOCKX ? i : 0] : BLOCKX ? o.c[s] * o.xv[i] : o.c[s];
        if (FAST) {
          facc[s][i] = __builtin_fmaf((float)S[s][i], m, facc[s][i]);
        } else {
          facc[s][i] = facc[s][i] + (float)S[s][i] * m;
        }
      }
  };

  // DEPTH register sets; block b lives in set b % DEPTH (named by the unrolled index). A group's
  // MFMAs are issued back to back (they do not depend on one another's rescale), then rescaled in
  // block order; blocks past the last are neither accumulated nor rescaled (uniform branches).
  Ops ops[DEPTH];
#pragma unroll
  for (int k = 0; k < DEPTH; ++k) load(k, ops[k]);
  for (int b0 = 0; b0 < nb; b0 += DEPTH) {
    if (TOK && WDT == WQ8) {
#pragma unroll
      for (int k = 0; k < DEPTH; ++k) {
        if (b0 + k < nb)
#pragma unroll
          for (int s = 0; s < NSEL; ++s) iacc[s] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ops[k].A, ops[k].B[s], iacc[s], 0, 0, 0);
        load(b0 + k + DEPTH, ops[k]);  // unconditional (clamped): exact wait counts
      }
    } else {
      v16i S[DEPTH][NSEL];
#pragma unroll
      for (int k = 0; k < DEPTH; ++k) sums(ops[k], S[k]);
#pragma unroll
      for (int k = 0; k < DEPTH; ++k) {
        if (b0 + k < nb) rescale(ops[k], S[k]);
        load(b0 + k + DEPTH, ops[k]);
      }
    }
  }

  // epilogue: row r0 + l32 (lane), tokens t0 + 8 (i / 4) + 4 h + i % 4 (accumulator i)
  const int r = r0 + l32;
  const int rc = min(r, tg.N - 1);
  const int tv = min(kWaveTile, a.T - t0);
  const uint32_t tbytes = (uint32_t)tv * (uint32_t)tg.N * 4u;
  const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(tg.y + (int64_t)t0 * tg.N, (short)0, (int)tbytes, 0x00020000);
  const int tb = 4 * h;
  float xt[16];
  if (TOK) {
    float* xdt = xdt_all + wave * 32;
    if (lane < 32) xdt[lane] = a.xd[t0 + lane];
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < 16; ++i) xt[i] = xdt[tb + 8 * (i >> 2) + (i & 3)];
  }
  auto value = [&](int s, int i, float ws) {
    if (WDT == WQ8) return TOK ? ((float)iacc[s][i] * xt[i]) * ws : facc[s][i] * ws;
    return TOK ? (facc[s][i] * 0.0625f) * xt[i] : facc[s][i] * 0.0625f;
  };
  if (SW) {
    // gate and up through this wave's LDS slice, so that silu (an expf) is emitted once in a loop
    float* const ep = ep_all + wave * (2 * 32 * 32);
    const float ws = WDT == WQ8 ? tg.scales[rc] : 1.f;
    const float wsu = WDT == WQ8 ? a.tg[1].scales[rc] : 1.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      ep[i * 64 + lane] = value(0, i, ws);
      ep[1024 + i * 64 + lane] = value(NSEL - 1, i, wsu);
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll 1
    for (int i = 0; i < 16; ++i) {
      const int t = tb + 8 * (i >> 2) + (i & 3);
      const float out = silu_exact(ep[i * 64 + lane]) * ep[1024 + i * 64 + lane];
      const int off = r < tg.N ? (t * tg.N + r) * 4 : 0x7FFFFFF0;
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, out), ry, off, 0, 0);
    }
    return;
  }
  const float ws = WDT == WQ8 ? tg.scales[rc] : 1.f;
  const bool has_res = tg.res != nullptr;
  const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(has_res ? tg.res + (int64_t)t0 * tg.N : tg.y), (short)0, has_res ? (int)tbytes : 0, 0x00020000);
  float res[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int t = tb + 8 * (i >> 2) + (i & 3);
    const int off = r < tg.N ? (t * tg.N + r) * 4 : 0x7FFFFFF0;
    res[i] = has_res ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, off, 0, 0)) : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int t = tb + 8 * (i >> 2) + (i & 3);
    const int off = r < tg.N ? (t * tg.N + r) * 4 : 0x7FFFFFF0;
    float out = value(0, i, ws);
    if (has_res) out = out + res[i];
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, out), ry, off, 0, 0);
  }
}

// The same per-wave scheme with 16 x 16 tiles (v_mfma_i32_16x16x32_i8: lane l supplies row
// l % 16 of A and column l % 16 of B, K elements 8 (l / 16) .. + 7 each, and holds
// D[4 (l / 16) + i][l % 16]). A quarter of the outputs per wave: four times the waves on a
// problem, and a quarter of the per-block rescale, the serial part of a wave (one dependent
// convert-multiply-add per output and block). Used when 32 x 32 waves would not fill the chip.
constexpr int kWave16 = 16;

template <int WDT, bool SW, bool TOK>
struct Wave16Ops {
  static constexpr int NSEL = SW ? 2 : 1;
  static constexpr bool BLOCKX = !TOK;
  long A;
  long B[NSEL];
  float c[NSEL];               // q4: ws of the lane's row and block
  float4 xv;                   // block scales of the lane's 4 tokens
};

__device__ __forceinline__ long q4_operand8(uint2 w, int h) {
  const int sh = 4 - 4 * h;
  const uint32_t lo = ((w.x << sh) & 0xF0F0F0F0u) ^ 0x80808080u, hi = ((w.y << sh) & 0xF0F0F0F0u) ^ 0x80808080u;
  return (long)(((uint64_t)hi << 32) | lo);
}

// The epilogue of a 16 x 16 wave tile (gemm_wave16_kernel, gemm_lds16_kernel): row r0 + l16,
// tokens t0 + 4 c4 + i (accumulator i); the row (and token) rescale, then SwiGLU or the residual,
// stores bounded by T and N.
template <int WDT, bool SW, bool TOK>
__device__ __forceinline__ void wave16_store(const GemmArgs& a, const GemmTarget& tg, int r0, int t0, int lane,
                                             const v4i (&iacc)[SW ? 2 : 1], const float (&facc)[SW ? 2 : 1][4]) {
  constexpr int NSEL = SW ? 2 : 1;
  const int l16 = lane & 15, c4 = lane >> 4;
  const int r = r0 + l16;
  const int rc = min(r, tg.N - 1);
  const int tv = min(kWave16, a.T - t0);
  const uint32_t tbytes = (uint32_t)tv * (uint32_t)tg.N * 4u;
  const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(tg.y + (int64_t)t0 * tg.N, (short)0, (int)tbytes, 0x00020000);
  float xt[4] = {1.f, 1.f, 1.f, 1.f};
  if (TOK) {
#pragma unroll
    for (int i = 0; i < 4; ++i) xt[i] = a.xd[min(t0 + 4 * c4 + i, a.Tpad - 1)];
  }
  auto value = [&](int s, int i, float ws) {
    if (WDT == WQ8) return TOK ? ((float)iacc[s][i] * xt[i]) * ws : facc[s][i] * ws;
    return TOK ? (facc[s][i] * 0.0625f) * xt[i] : facc[s][i] * 0.0625f;
  };
  const float ws = WDT == WQ8 ? tg.scales[rc] : 1.f;
  if (SW) {
    const float wsu = WDT == WQ8 ? a.tg[1].scales[rc] : 1.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int off = r < tg.N ? ((4 * c4 + i) * tg.N + r) * 4 : 0x7FFFFFF0;
      const float out = silu_exact(value(0, i, ws)) * value(NSEL - 1, i, wsu);
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, out), ry, off, 0, 0);
    }
    return;
  }
  const bool has_res = tg.res != nullptr;
  const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(has_res ? tg.res + (int64_t)t0 * tg.N : tg.y), (short)0, has_res ? (int)tbytes : 0, 0x00020000);
  float res[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int off = r < tg.N ? ((4 * c4 + i) * tg.N + r) * 4 : 0x7FFFFFF0;
    res[i] = has_res ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, off, 0, 0)) : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int off = r < tg.N ? ((4 * c4 + i) * tg.N + r) * 4 : 0x7FFFFFF0;
    float out = value(0, i, ws);
    if (has_res) out = out + res[i];
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, out), ry, off, 0, 0);
  }
}

constexpr int kWave16Depth = 8;  // blocks in flight per wave (its operands are small)

template <int WDT, bool SW, bool TOK, bool FAST, int DEPTH = kWave16Depth>
__global__ __launch_bounds__(256) void gemm_wave16_kernel(const GemmArgs a) {
  typedef Wave16Ops<WDT, SW, TOK> Ops;
  constexpr int NSEL = Ops::NSEL;
  constexpr bool BLOCKX = Ops::BLOCKX;
  const int lane = threadIdx.x & 63, l16 = lane & 15, c4 = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int nb = a.nb, H = a.H;
  const int ngroups = (a.T + kWave16 - 1) / kWave16;
  // wave -> (target, 16-row tile, 16-token group), token group fastest
  int rt = (int)blockIdx.x * 4 + wave;
  const int g = rt % ngroups;
  rt /= ngroups;
  int ti = 0;
  const int n = SW ? 1 : a.n_targets;
  for (; ti < n; ++ti) {
    const int cnt = (a.tg[ti].N + kWave16 - 1) / kWave16;
    if (rt < cnt) break;
    rt -= cnt;
  }
  if (ti >= n) return;  // past the last tile (uniform per wave; no barrier below)
  const GemmTarget tg = SW ? a.tg[0] : gemm_target_at(ti);
  const int r0 = rt * kWave16, t0 = g * kWave16;
  const int rows_pad = (tg.N + kPadRows - 1) / kPadRows * kPadRows;
  const int wrow = min(r0 + l16, rows_pad - 1);
  const int64_t rbase = (int64_t)(wrow / H) * nb * H + (wrow % H);  // item of (wrow, block 0)
  const uint8_t* const wd[2] = {tg.data, SW ? a.tg[1].data : tg.data};
  const float* const wsc[2] = {tg.scales, SW ? a.tg[1].scales : tg.scales};
  // token t0 + l16 of the 32-token fragment (xq layout: lane h*32 + t%32 holds elements h*16 ..
  // h*16 + 15 of token t), elements 8 c4 .. 8 c4 + 7
  const int8_t* const xg = a.xq + (int64_t)(t0 >> 5) * nb * 1024 + ((c4 >> 1) * 32 + (t0 & 31) + l16) * 16 + (c4 & 1) * 8;

  auto load = [&](int blk, Ops& o) {
    blk = min(blk, nb - 1);
    o.A = *reinterpret_cast<const long*>(xg + (int64_t)blk * 1024);
    const int64_t it = rbase + (int64_t)blk * H;
#pragma unroll
    for (int s = 0; s < NSEL; ++s) {
      if (WDT == WQ8) {
        o.B[s] = *reinterpret_cast<const long*>(wd[s] + it * 32 + c4 * 8);
        o.c[s] = 1.f;
      } else {
        o.B[s] = q4_operand8(*reinterpret_cast<const uint2*>(wd[s] + it * 16 + (c4 & 1) * 8), c4 >> 1);
        o.c[s] = wsc[s][it];
      }
    }
    if (BLOCKX) o.xv = *reinterpret_cast<const float4*>(a.xd + (int64_t)blk * a.Tpad + t0 + 4 * c4);
  };

  v4i iacc[NSEL];
  float facc[NSEL][4];
  const v4i zero = {0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < NSEL; ++s) {
    iacc[s] = zero;
#pragma unroll
    for (int i = 0; i < 4; ++i) facc[s][i] = 0.f;
  }
  auto rescale = [&](const Ops& o, const v4i (&S)[NSEL]) {
    const float xv[4] = {o.xv.x, o.xv.y, o.xv.z, o.xv.w};
#pragma unroll
    for (int s = 0; s < NSEL; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // q8: p = float(S) * xd; q4 (S = 16 * S_b, c = ws): p = float(S) * (c * xd) = 16 * edgelm's product
        const float m = WDT == WQ8 ? xv[BLOCKX ? i : 0] : BLOCKX ? o.c[s] * xv[i] : o.c[s];
        if (FAST) {
          facc[s][i] = __builtin_fmaf((float)S[s][i], m, facc[s][i]);
        } else {
          facc[s][i] = facc[s][i] + (float)S[s][i] * m;
        }
      }
  };

  Ops ops[DEPTH];
#pragma unroll
  for (int k = 0; k < DEPTH; ++k) load(k, ops[k]);
  for (int b0 = 0; b0 < nb; b0 += DEPTH) {
    if (TOK && WDT == WQ8) {
#pragma unroll
      for (int k = 0; k < DEPTH; ++k) {
        if (b0 + k < nb)
#pragma unroll
          for (int s = 0; s < NSEL; ++s) iacc[s] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ops[k].A, ops[k].B[s], iacc[s], 0, 0, 0);
        load(b0 + k + DEPTH, ops[k]);  // unconditional (clamped): exact wait counts
      }
    } else {
      v4i S[DEPTH][NSEL];
#pragma unroll
      for (int k = 0; k < DEPTH; ++k)
#pragma unroll
        for (int s = 0; s < NSEL; ++s) S[k][s] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ops[k].A, ops[k].B[s], zero, 0, 0, 0);
#pragma unroll
      for (int k = 0; k < DEPTH; ++k) {
        if (b0 + k < nb) rescale(ops[k], S[k]);
        load(b0 + k + DEPTH, ops[k]);
      }
    }
  }

  wave16_store<WDT, SW, TOK>(a, tg, r0, t0, lane, iacc, facc);
}

// Small GEMMs (K <= 1536: the prefill of a small model): gemm_wave16_kernel's waves and arithmetic
// (the same bits), with a workgroup's operands (one 16-row tile, 64 tokens: four waves of 16
// tokens) moved into LDS by DMA in one go, 1 KB per instruction, every request out before the
// first wait: the activation fragments of the 64 tokens (two 32-token groups, contiguous in xq),
// their block scales, the 16 rows' weight items and their q4 scales. gemm_wave16_kernel loads each
// wave's operands from L2 eight blocks ahead, and its loop is bound by that latency (~150 ns per
// 32-block with the operands in the Infinity Cache, measured at T = 128, K = 1536); here the loop
// reads LDS. LDS: A [TW/32][nb][1024] | XD [nb][TW] f32 (token mode: [64]) | B[s] [nb][RW][G] |
// BS[s] (q4) [nb][RW] f32, each region with room for kLds16Ahead more blocks and rounded up to 1 KB
// (gemm_lds16_bytes).
// QF (SwiGLU in block mode, the quantized-h handoff): a workgroup is 32 rows x 32 tokens instead
// (wave w: rows 16 (w & 1) .., tokens 16 (w >> 1) ..), so it holds whole 32-blocks of h; after the
// stores, the two waves of a token group exchange their 16-row amax through LDS and each writes its
// half of every block into the next GEMM's fragments with edgelm's rounding (act_quant_frag_kernel's
// arithmetic: s = amax / 127, each value's rounding that of its division).
__host__ __device__ constexpr int lds16_region_bytes(int bytes) { return (bytes + 1023) / 1024 * 1024; }
constexpr int kLds16MaxBlocks = 48;  // K <= 1536
constexpr int kLds16Ahead = 3;       // blocks read ahead; every region has room for them past nb
template <int WDT, bool SW, bool TOK, bool QF = false>
__host__ __device__ inline int gemm_lds16_bytes(int nb) {
  constexpr int G = WDT == WQ8 ? 32 : 16, NSEL = SW ? 2 : 1, P = kLds16Ahead;
  constexpr int RW = QF ? 32 : 16, TW = QF ? 32 : 64;
  const int xd = TOK ? 1024 : lds16_region_bytes((nb + P) * TW * 4);
  const int bw = lds16_region_bytes((nb + P) * RW * G), bs = WDT == WQ4 ? lds16_region_bytes((nb + P) * RW * 4) : 0;
  return (TW / 32 * nb + P) * 1024 + xd + NSEL * (bw + bs) + (QF ? 1024 : 0);
}

template <int WDT, bool SW, bool TOK, bool FAST, bool QF, bool MT>
__global__ __launch_bounds__(256) void gemm_lds16_kernel(const GemmArgs a) {
  static_assert(!QF || (SW && !TOK), "quantized h: SwiGLU in block mode");
  // every launch argument the kernel reads, in scalar registers first, through one asm statement (loads
  // feeding one statement go out as one batch: one round trip to the argument segment; the GEMVs do
  // the same). MT: more than one target (a fused QKV).
  // (T goes through the statement, so that the tile arithmetic on it cannot start before it)
  int Ta = a.T;
  // MT: every target's fields, pinned through the statement, so that the target is picked by selects
  // instead of a second load at its index
  const uint8_t *d0 = a.tg[0].data, *d1 = a.tg[1].data, *d2 = a.tg[2].data, *d3 = a.tg[3].data;
  const float *s0 = a.tg[0].scales, *s1 = a.tg[1].scales, *s2 = a.tg[2].scales, *s3 = a.tg[3].scales;
  float *y0 = a.tg[0].y, *y1 = a.tg[1].y, *y2 = a.tg[2].y, *y3 = a.tg[3].y;
  const float *q0 = a.tg[0].res, *q1 = a.tg[1].res, *q2 = a.tg[2].res, *q3 = a.tg[3].res;
  if constexpr (MT)
    asm volatile(""
                 : "+s"(Ta), "+s"(d0), "+s"(d1), "+s"(d2), "+s"(d3), "+s"(s0), "+s"(s1), "+s"(s2), "+s"(s3), "+s"(y0),
                   "+s"(y1), "+s"(y2), "+s"(y3), "+s"(q0), "+s"(q1), "+s"(q2), "+s"(q3)
                 : "s"(a.xq), "s"(a.xd), "s"(a.Tpad), "s"(a.nb), "s"(a.H), "s"(a.n_targets), "s"(a.tg[0].N),
                   "s"(a.tg[1].N), "s"(a.tg[2].N), "s"(a.tg[3].N));
  else if constexpr (QF)
    asm volatile("" : "+s"(Ta) : "s"(a.xq), "s"(a.xd), "s"(a.Tpad), "s"(a.nb), "s"(a.H), "s"(a.tg[0].N),
                 "s"(a.tg[0].data), "s"(a.tg[0].scales), "s"(a.tg[0].y), "s"(a.tg[1].data), "s"(a.tg[1].scales),
                 "s"(a.oq), "s"(a.od), "s"(a.onb));
  else if constexpr (SW)
    asm volatile("" : "+s"(Ta) : "s"(a.xq), "s"(a.xd), "s"(a.Tpad), "s"(a.nb), "s"(a.H), "s"(a.tg[0].N),
                 "s"(a.tg[0].data), "s"(a.tg[0].scales), "s"(a.tg[0].y), "s"(a.tg[1].data), "s"(a.tg[1].scales));
  else
    asm volatile("" : "+s"(Ta) : "s"(a.xq), "s"(a.xd), "s"(a.Tpad), "s"(a.nb), "s"(a.H), "s"(a.tg[0].N),
                 "s"(a.tg[0].data), "s"(a.tg[0].scales), "s"(a.tg[0].y), "s"(a.tg[0].res));
  typedef Wave16Ops<WDT, SW, TOK> Ops;
  constexpr int NSEL = Ops::NSEL, G = WDT == WQ8 ? 32 : 16;
  constexpr bool BLOCKX = Ops::BLOCKX;
  constexpr int RW = QF ? 32 : 16, TW = QF ? 32 : 64;  // rows and tokens of a workgroup
  extern __shared__ __align__(16) unsigned char lds[];
  const int lane = threadIdx.x & 63, l16 = lane & 15, c4 = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int rh = QF ? wave & 1 : 0, tgw = QF ? wave >> 1 : wave;  // the wave's row half, token group
  const int nb = a.nb, H = a.H;
  // workgroup -> (target, RW-row tile, TW-token chunk), chunk fastest
  const int nchunk = (Ta + TW - 1) / TW;
  int rt = (int)blockIdx.x;
  const int ch = rt % nchunk;
  rt /= nchunk;
  // the target: with one, the first; with more, from every target's tile count (N's read in the
  // first batch), then its fields at its index
  const int n = MT ? a.n_targets : 1;
  const int e1 = (pin_sgpr(a.tg[0].N) + RW - 1) / RW;
  const int e2 = MT ? e1 + (pin_sgpr(a.tg[1].N) + RW - 1) / RW : e1;
  const int e3 = MT ? e2 + (pin_sgpr(a.tg[2].N) + RW - 1) / RW : e2;
  const int e4 = MT ? e3 + (pin_sgpr(a.tg[3].N) + RW - 1) / RW : e3;
  const int ti = (rt >= e1) + (n > 1 && rt >= e2) + (n > 2 && rt >= e3) + (n > 3 && rt >= e4);
  if (ti >= n) return;  // past the last tile (uniform per workgroup; no barrier below)
  rt -= ti == 0 ? 0 : ti == 1 ? e1 : ti == 2 ? e2 : e3;
  GemmTarget tg;
  if constexpr (MT) {
    tg.data = pin_global(ti == 0 ? d0 : ti == 1 ? d1 : ti == 2 ? d2 : d3);
    tg.scales = pin_global(ti == 0 ? s0 : ti == 1 ? s1 : ti == 2 ? s2 : s3);
    tg.y = pin_global(ti == 0 ? y0 : ti == 1 ? y1 : ti == 2 ? y2 : y3);
    tg.res = pin_global(ti == 0 ? q0 : ti == 1 ? q1 : ti == 2 ? q2 : q3);
    tg.N = ti == 0 ? a.tg[0].N : ti == 1 ? a.tg[1].N : ti == 2 ? a.tg[2].N : a.tg[3].N;
    tg.ntiles = 0;  // not read here
  } else {
    tg = a.tg[0];
  }
  const int r0 = rt * RW, tc = ch * TW;
  const uint8_t* const wd[2] = {tg.data, SW ? a.tg[1].data : tg.data};
  const float* const wsc[2] = {tg.scales, SW ? a.tg[1].scales : tg.scales};
  constexpr int P = kLds16Ahead;
  const int xd_bytes = TOK ? 1024 : lds16_region_bytes((nb + P) * TW * 4);
  const int bw_bytes = lds16_region_bytes((nb + P) * RW * G);
  const int bs_bytes = WDT == WQ4 ? lds16_region_bytes((nb + P) * RW * 4) : 0;
  unsigned char* const A = lds;
  unsigned char* const XD = A + (TW / 32 * nb + P) * 1024;
  unsigned char* const BW = XD + xd_bytes;             // [s] at BW + s * bw_bytes
  unsigned char* const BS = BW + NSEL * bw_bytes;      // [s] at BS + s * bs_bytes
  const unsigned base = (unsigned)(size_t)(LdsBytes)lds;
  const unsigned xd_lds = base + (TW / 32 * nb + P) * 1024, bw_lds = xd_lds + xd_bytes, bs_lds = bw_lds + NSEL * bw_bytes;

  // 1. every operand of the workgroup into LDS; instruction j of a region fills its KB j, and wave w
  // issues j = w, w + 4, ... Chunks past a region's end repeat its last one (into the padding).
  {
    // activation fragments: the token groups are contiguous in xq ([Tpad/32][nb][1 KB])
    const int8_t* const xs = a.xq + (int64_t)(tc >> 5) * nb * 1024;
    for (int j = wave; j < TW / 32 * nb; j += 4) dma16s(xs, (uint32_t)(j * 1024 + lane * 16), base + j * 1024);
    if (BLOCKX) {  // XD[b][t]: TW / 4 lanes per block (4 tokens each), 256 / TW blocks per instruction
      constexpr int LPB = TW / 4, BPI = 64 / LPB;
      for (int j = wave; BPI * j < nb; j += 4) {
        const int b = min(BPI * j + lane / LPB, nb - 1);
        dma16s(a.xd, (uint32_t)(((int64_t)b * a.Tpad + tc + 4 * (lane % LPB)) * 4), xd_lds + j * 1024);
      }
    } else if (wave == 0) {  // XD[t]
      dma16s(a.xd, (uint32_t)((tc + 4 * l16) * 4), xd_lds);
    }
    // weight item (row, b) sits at ((row / H) nb + b) H + row % H (H a power of two; the launch
    // keeps byte offsets below 2^31)
    const int lgH = __builtin_ctz(H);
    auto item = [&](int row, int b) { return (((row >> lgH) * nb + b) << lgH) + (row & (H - 1)); };
    constexpr int CPB = RW * G / 16;  // 16-byte chunks per block of the RW rows
    const int nw = nb * CPB;
#pragma unroll
    for (int s = 0; s < NSEL; ++s) {
      for (int j = wave; 64 * j < nw; j += 4) {
        const int c = min(64 * j + lane, nw - 1), b = c / CPB, w = c - b * CPB;
        const int row = WDT == WQ8 ? w >> 1 : w, half = WDT == WQ8 ? (w & 1) : 0;
        dma16s(wd[s], (uint32_t)(item(r0 + row, b) * G + half * 16), bw_lds + s * bw_bytes + j * 1024);
      }
      if (WDT == WQ4) {  // BS[b][row]: 4 rows per chunk, consecutive items (H >= 4, r0 % 4 == 0)
        constexpr int QPB = RW / 4;
        const int ns = nb * QPB;
        for (int j = wave; 64 * j < ns; j += 4) {
          const int c = min(64 * j + lane, ns - 1), b = c / QPB, q = c - b * QPB;
          dma16s(wsc[s], (uint32_t)(item(r0 + 4 * q, b) * 4), bs_lds + s * bs_bytes + j * 1024);
        }
      }
    }
    wait_vm<0>();
    __syncthreads();
  }

  // 2. the wave's 16 tokens against its 16 rows, block by block from LDS, D blocks read ahead
  const int tw = tgw * kWave16, t0 = tc + tw, rw0 = rh * 16;
  const unsigned char* const xa = A + (tw >> 5) * nb * 1024 + ((c4 >> 1) * 32 + (tw & 31) + l16) * 16 + (c4 & 1) * 8;
  auto load = [&](int blk, Ops& o) {
    // blocks nb .. nb + P - 1 (read ahead, never used) lie in the regions' padding
    o.A = *reinterpret_cast<const long*>(xa + blk * 1024);
#pragma unroll
    for (int s = 0; s < NSEL; ++s) {
      const unsigned char* const bw = BW + s * bw_bytes + (blk * RW + rw0 + l16) * G;
      if (WDT == WQ8) {
        o.B[s] = *reinterpret_cast<const long*>(bw + c4 * 8);
        o.c[s] = 1.f;
      } else {
        o.B[s] = q4_operand8(*reinterpret_cast<const uint2*>(bw + (c4 & 1) * 8), c4 >> 1);
        o.c[s] = reinterpret_cast<const float*>(BS + s * bs_bytes)[blk * RW + rw0 + l16];
      }
    }
    if (BLOCKX) o.xv = *reinterpret_cast<const float4*>(XD + (blk * TW + tw + 4 * c4) * 4);
  };
  v4i iacc[NSEL];
  float facc[NSEL][4];
  const v4i zero = {0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < NSEL; ++s) {
    iacc[s] = zero;
#pragma unroll
    for (int i = 0; i < 4; ++i) facc[s][i] = 0.f;
  }
  auto rescale = [&](const Ops& o, const v4i (&S)[NSEL]) {
    const float xv[4] = {o.xv.x, o.xv.y, o.xv.z, o.xv.w};
#pragma unroll
    for (int s = 0; s < NSEL; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float m = WDT == WQ8 ? xv[BLOCKX ? i : 0] : BLOCKX ? o.c[s] * xv[i] : o.c[s];
        if (FAST) {
          facc[s][i] = __builtin_fmaf((float)S[s][i], m, facc[s][i]);
        } else {
          facc[s][i] = facc[s][i] + (float)S[s][i] * m;
        }
      }
  };
  // Straight-line code over the blocks (at most kLds16MaxBlocks): block k + 3's operands are read
  // and block k + 1's MFMA issued before block k's products are rescaled and added, every read
  // unconditional once its step is reached (the empty asm keeps the compiler from sinking it past
  // the exits), so the operands of an MFMA were requested two steps before. (In a loop the
  // compiler's wait-count pass made every iteration wait for all reads at its head.)
  Ops ops[4];
  v4i S[2][NSEL];
  load(0, ops[0]);
  load(1, ops[1]);
  load(2, ops[2]);
  asm volatile("" ::: "memory");
  if (!(TOK && WDT == WQ8)) {
#pragma unroll
    for (int s = 0; s < NSEL; ++s) S[0][s] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ops[0].A, ops[0].B[s], zero, 0, 0, 0);
  }
#define ELM_L16_STEP(k)                                                                                   \
  if (nb <= (k)) goto done;                                                                              \
  if ((k) + 3 < kLds16MaxBlocks) {                                                                       \
    load((k) + 3, ops[((k) + 3) % 4]);                                                                   \
    asm volatile("" ::: "memory");                                                                       \
    __builtin_amdgcn_sched_barrier(0);                                                                   \
  }                                                                                                      \
  if (TOK && WDT == WQ8) {                                                                               \
    _Pragma("unroll") for (int s = 0; s < NSEL; ++s) iacc[s] =                                           \
        __builtin_amdgcn_mfma_i32_16x16x32_i8(ops[(k) % 4].A, ops[(k) % 4].B[s], iacc[s], 0, 0, 0);       \
  } else {                                                                                               \
    if ((k) + 1 < kLds16MaxBlocks) {                                                                     \
      _Pragma("unroll") for (int s = 0; s < NSEL; ++s) S[((k) + 1) % 2][s] =                             \
          __builtin_amdgcn_mfma_i32_16x16x32_i8(ops[((k) + 1) % 4].A, ops[((k) + 1) % 4].B[s], zero, 0, 0, 0); \
    }                                                                                                    \
    rescale(ops[(k) % 4], S[(k) % 2]);                                                                   \
  }
  ELM_L16_STEP(0) ELM_L16_STEP(1) ELM_L16_STEP(2) ELM_L16_STEP(3) ELM_L16_STEP(4) ELM_L16_STEP(5)
  ELM_L16_STEP(6) ELM_L16_STEP(7) ELM_L16_STEP(8) ELM_L16_STEP(9) ELM_L16_STEP(10) ELM_L16_STEP(11)
  ELM_L16_STEP(12) ELM_L16_STEP(13) ELM_L16_STEP(14) ELM_L16_STEP(15) ELM_L16_STEP(16) ELM_L16_STEP(17)
  ELM_L16_STEP(18) ELM_L16_STEP(19) ELM_L16_STEP(20) ELM_L16_STEP(21) ELM_L16_STEP(22) ELM_L16_STEP(23)
  ELM_L16_STEP(24) ELM_L16_STEP(25) ELM_L16_STEP(26) ELM_L16_STEP(27) ELM_L16_STEP(28) ELM_L16_STEP(29)
  ELM_L16_STEP(30) ELM_L16_STEP(31) ELM_L16_STEP(32) ELM_L16_STEP(33) ELM_L16_STEP(34) ELM_L16_STEP(35)
  ELM_L16_STEP(36) ELM_L16_STEP(37) ELM_L16_STEP(38) ELM_L16_STEP(39) ELM_L16_STEP(40) ELM_L16_STEP(41)
  ELM_L16_STEP(42) ELM_L16_STEP(43) ELM_L16_STEP(44) ELM_L16_STEP(45) ELM_L16_STEP(46) ELM_L16_STEP(47)
#undef ELM_L16_STEP
done:
  if constexpr (QF) {
    // h for tokens t0 + 4 c4 + i, row r0 + rw0 + l16, as wave16_store forms and stores it (tokens past
    // T were computed from the padding's fragments; nothing stores them but the fragments, which the
    // next GEMM never stores either)
    const int r = r0 + rw0 + l16, rc = min(r, tg.N - 1);
    const float ws = WDT == WQ8 ? tg.scales[rc] : 1.f, wsu = WDT == WQ8 ? a.tg[1].scales[rc] : 1.f;
    float hv[4], am[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // q8 facc * ws, q4 facc / 16, then silu(gate) * up
      const float g = WDT == WQ8 ? facc[0][i] * ws : facc[0][i] * 0.0625f;
      const float u = WDT == WQ8 ? facc[1][i] * wsu : facc[1][i] * 0.0625f;
      hv[i] = silu_exact(g) * u;
    }
    if (t0 < a.T) {  // wave-uniform; the stores bounded by T and N as in wave16_store
      const int tv = min(kWave16, a.T - t0);
      const uint32_t tbytes = (uint32_t)tv * (uint32_t)tg.N * 4u;
      const __amdgpu_buffer_rsrc_t ry =
          __builtin_amdgcn_make_buffer_rsrc(tg.y + (int64_t)t0 * tg.N, (short)0, (int)tbytes, 0x00020000);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int off = r < tg.N ? ((4 * c4 + i) * tg.N + r) * 4 : 0x7FFFFFF0;
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, hv[i]), ry, off, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // the amax over the wave's 16 rows (the 16 lanes of each row of the wave)
      float v = fabsf(hv[i]);
      v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
      v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
      v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
      am[i] = fmaxf(v, dpp_f<kDppRowMirror>(v));
    }
    float* const ex = reinterpret_cast<float*>(BS + NSEL * bs_bytes);  // [token group][row half][16 tokens]
    if (l16 == 0)
#pragma unroll
      for (int i = 0; i < 4; ++i) ex[(tgw * 2 + rh) * 16 + 4 * c4 + i] = am[i];
    lds_barrier();  // the partner wave's amax is in LDS (the h stores stay in flight)
    const int b = r0 / kBlock;  // the workgroup's 32 rows are block b of h
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float amax = fmaxf(am[i], ex[(tgw * 2 + (rh ^ 1)) * 16 + 4 * c4 + i]);
      const float d = amax / 127.0f;
      int q;
      elm_q8_group<1>(&hv[i], d == 0.f ? 1.f : d, &q);
      const int t = t0 + 4 * c4 + i;
      if (r0 + rw0 + l16 < tg.N && t < a.Tpad) {
        a.oq[elm_frag_offset(t, b, rh, a.onb) + l16] = (int8_t)q;
        if (l16 == 0 && rh == 0) a.od[(int64_t)b * a.Tpad + t] = d;
      }
    }
  } else {
    if (t0 < a.T) wave16_store<WDT, SW, TOK>(a, tg, r0, t0, lane, iacc, facc);
  }
}

// ---------------------------------------------------------------- f32-activation paths

// The target owning tile `tile` of an f32-activation launch (tile made relative to it): the target
// count and the tile starts, pinned in scalar registers, come with the kernel's other arguments in
// one batch of scalar loads; the target's fields then take one more (uniform) load through the
// argument segment, instead of the tile starts one per step of a search and an indexed copy.
template <bool SW>
__device__ __forceinline__ GemvTarget f32_target(const F32Args& a, int& tile) {
  if (SW) return a.tg[0];
  // one statement pins the lookup's values and takes the kernels' other arguments as inputs, so that
  // all of their loads go out together
  int n = a.n_targets, ts0 = a.tile_start[0], ts1 = a.tile_start[1], ts2 = a.tile_start[2], ts3 = a.tile_start[3];
  asm volatile("" : "+s"(n), "+s"(ts0), "+s"(ts1), "+s"(ts2), "+s"(ts3)
               : "s"(a.H), "s"(a.x), "s"(a.T), "s"(a.K), "s"(a.nb), "s"(a.nw), "s"(a.eps), "s"(a.rt));
  const int ti = (n > 1 && tile >= ts1) + (n > 2 && tile >= ts2) + (n > 3 && tile >= ts3);
  tile -= ti == 0 ? ts0 : ti == 1 ? ts1 : ti == 2 ? ts2 : ts3;
  typedef const F32Args __attribute__((address_space(4)))* KernArgs;
  const KernArgs ka = (KernArgs)__builtin_amdgcn_kernarg_segment_ptr();
  GemvTarget t;
  t.data = pin_global(ka->tg[ti].data);
  t.scales = pin_global(ka->tg[ti].scales);
  t.y = pin_global(ka->tg[ti].y);
  t.res = pin_global(ka->tg[ti].res);
  t.N = ka->tg[ti].N;
  t.tiles = ka->tg[ti].tiles;
  return t;
}


// T == 1, q4, one workgroup per H-row tile (of the target, or of gate and up with SW): dot_q4's
// operations (kernels_cpu.cpp:397-399) spread over the groups instead of one lane walking the row.
// Every (selection, row, group) item is (g0 + g1) * ws_g, g0 / g1 the in-order 16-term sums of the
// group's low / high nibbles against x, and goes to LDS; then one lane per row adds its row's items
// in group order (s = s + p_g from s = 0, as dot_q4 does) and applies the epilogue.
// With a.nw, x is first RMSNORM'd in the workgroup in rmsnorm_kernel's float order (four strided
// sums of squares, (s0 + s1) + (s2 + s3), inv = 1 / sqrt(ss / K + eps), (x * inv) * w), so that
// RMSNORM and the matmul after it take one launch.
template <bool SW>
__global__ __launch_bounds__(256) void gemv_f32act_q4_kernel(const F32Args a) {
  extern __shared__ __align__(16) float f32q4_lds[];
  __shared__ float inv_s;
  constexpr int NSEL = SW ? 2 : 1;
  const int K = a.K, nb = a.nb, H = a.H, RT = a.rt, lgRT = __builtin_ctz(RT), pst = nb + 1;
  float* const sx = f32q4_lds;                // [K]
  float* const P = f32q4_lds + ((K + 3) & ~3);  // [NSEL][RT][nb + 1]
  int tile = blockIdx.x;
  const GemvTarget tg = f32_target<SW>(a, tile);
  const int per_sel = RT * nb, items = NSEL * per_sel, n0 = tile * RT;
  const int64_t ibase = (int64_t)(n0 / H) * nb * H + n0 % H;  // item (row n0, group 0)
  // the first item's weights go out before x is staged, so that the two loads overlap
  const auto item_of = [&](int it, int& sel, int& g, int& r) -> int64_t {
    sel = SW && it >= per_sel ? 1 : 0;
    const int j = it - sel * per_sel;
    g = j >> lgRT;
    r = j & (RT - 1);
    return ibase + (int64_t)g * H + r;  // rows past N: the padding's items
  };
  uint4 wq0 = make_uint4(0, 0, 0, 0);
  float ws0 = 0.f;
  if ((int)threadIdx.x < items) {
    int sel, g, r;
    const int64_t item = item_of(threadIdx.x, sel, g, r);
    wq0 = *reinterpret_cast<const uint4*>((sel ? a.tg[1].data : tg.data) + item * 16);
    ws0 = (sel ? a.tg[1].scales : tg.scales)[item];
  }
  for (int i = threadIdx.x; i < K; i += 256) sx[i] = a.x[i];
  if (a.nw) {
    // squares as [accumulator][rowlen] (zero-padded: adding +0.0 to a sum of squares changes
    // nothing); K % 4 == 0 here (K = 32 nb)
    float* const sq = f32q4_lds + ((((K + 3) & ~3) + NSEL * RT * pst + 3) & ~3);
    const int K4 = K >> 2, rowlen = norm_rowlen(K), n16 = (K4 + 15) & ~15;
    for (int i = threadIdx.x; i < 4 * n16; i += 256) {
      const int c = i / n16, j = i - c * n16;
      const float v = j < K4 ? a.x[4 * j + c] : 0.f;
      sq[c * rowlen + j] = v * v;
    }
    __syncthreads();
    if (threadIdx.x < 4) {
      const float s = ordered_sum(sq + threadIdx.x * rowlen, K4, 0.f);
      const float s01 = s + dpp_f<kDppQuadXor1>(s);  // lane 0: s0 + s1, lane 2: s2 + s3
      const float ss = s01 + dpp_f<kDppQuadXor2>(s01);
      if (threadIdx.x == 0) inv_s = 1.0f / sqrtf(ss / (float)K + a.eps);
    }
    __syncthreads();
    const float inv = inv_s;
    for (int i = threadIdx.x; i < K; i += 256) sx[i] = (sx[i] * inv) * a.nw[i];
  }
  __syncthreads();
  for (int it = threadIdx.x; it < items; it += 256) {
    int sel, g, r;
    const int64_t item = item_of(it, sel, g, r);
    uint4 wq = wq0;
    float ws = ws0;
    if (it != (int)threadIdx.x) {
      wq = *reinterpret_cast<const uint4*>((sel ? a.tg[1].data : tg.data) + item * 16);
      ws = (sel ? a.tg[1].scales : tg.scales)[item];
    }
    const uint32_t wd[4] = {wq.x, wq.y, wq.z, wq.w};
    const float* const xs = sx + g * 32;
    float g0 = 0.f, g1 = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t byte = (wd[i >> 2] >> (8 * (i & 3))) & 0xFF;
      g0 = g0 + xs[i] * (float)((int)(byte & 0x0F) - 8);
      g1 = g1 + xs[16 + i] * (float)((int)(byte >> 4) - 8);
    }
    P[(sel * RT + r) * pst + g] = (g0 + g1) * ws;
  }
  __syncthreads();
  if ((int)threadIdx.x < RT) {
    const int r = threadIdx.x, n = n0 + r;
    if (n < tg.N) {
      const float* const pr = P + r * pst;
      float s = 0.f;
      for (int g = 0; g < nb; ++g) s = s + pr[g];
      if (SW) {
        const float* const pu = P + (RT + r) * pst;
        float u = 0.f;
        for (int g = 0; g < nb; ++g) u = u + pu[g];
        tg.y[n] = silu_exact(s) * u;
      } else {
        tg.y[n] = (tg.res ? tg.res[n] : 0.f) + s;
      }
    }
  }
}

// T == 1, q8, rows whose products fit the launch's 64 KB of LDS (x plus [sel][8 rows][4 chains][stride]
// floats: K up to 1792 for one output, up to 768 for SwiGLU; longer rows take the four-lane kernels
// below): the products x_i * w_i (each rounded, as dot_q8 forms
// them) are independent, so all 256 threads form them into LDS by chain ([sel][row][chain][K / 4],
// rows padded by 4 floats against bank conflicts); then lane 4r + c of wave 0 adds chain c of row
// r in order (the K mod 4 tail into chain 0) and ((s0 + s1) + (s2 + s3)) * ws follows. The
// dependent adds are all that stays on one lane. Eight rows per workgroup.
constexpr int kQ8PRows = 8;
__host__ __device__ inline int q8p_stride(int K) { return ((((K & ~3) >> 2) + 63) & ~63) + 4; }
template <bool SW>
__global__ __launch_bounds__(256) void gemv_f32act_q8_prod_kernel(const F32Args a) {
  extern __shared__ __align__(16) float q8p_lds[];
  constexpr int NSEL = SW ? 2 : 1;
  const int K = a.K, K4 = K & ~3, Lq = K4 >> 2, Lr = q8p_stride(K), H = a.H, nb = a.nb, tid = threadIdx.x;
  int grp = blockIdx.x;
  const GemvTarget tg = f32_target<SW>(a, grp);
  const int n0 = grp * kQ8PRows;  // rows past N: padding (rows_pad % 64 == 0)
  float* const sx = q8p_lds;
  float* const P = q8p_lds + ((K + 3) & ~3);  // [NSEL][kQ8PRows][4][Lr]
  for (int i = tid; i < K; i += 256) sx[i] = a.x[i];
  __syncthreads();
  for (int it = tid; it < NSEL * kQ8PRows * Lq; it += 256) {
    const int sr = it / Lq, q = it - sr * Lq, sel = sr / kQ8PRows, r = sr - sel * kQ8PRows, n = n0 + r;
    const int64_t item = (int64_t)(n / H) * nb * H + (int64_t)(q >> 3) * H + (n % H);
    const uint32_t w = *reinterpret_cast<const uint32_t*>((SW && sel ? a.tg[1].data : tg.data) + item * 32 + ((4 * q) & 31));
    float* const pr = P + (size_t)sr * 4 * Lr + q;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) pr[cc * Lr] = sx[4 * q + cc] * (float)(int8_t)((w >> (8 * cc)) & 0xFF);
  }
  __syncthreads();
  if (tid >= 4 * kQ8PRows) return;
  const int r = tid >> 2, c = tid & 3, n = n0 + r;
  const float* const rg = P + (size_t)(r * 4 + c) * Lr;
  const float* const ru = P + (size_t)((kQ8PRows + r) * 4 + c) * Lr;
  float sg = 0.f, su = 0.f;
  int j = 0;
  for (; j + 32 <= Lq; j += 32) {
    float4 vg[8], vu[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      vg[u] = *reinterpret_cast<const float4*>(rg + j + 4 * u);
      if (SW) vu[u] = *reinterpret_cast<const float4*>(ru + j + 4 * u);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      sg = sg + vg[u].x;
      sg = sg + vg[u].y;
      sg = sg + vg[u].z;
      sg = sg + vg[u].w;
      if (SW) {
        su = su + vu[u].x;
        su = su + vu[u].y;
        su = su + vu[u].z;
        su = su + vu[u].w;
      }
    }
  }
  for (; j < Lq; ++j) {
    sg = sg + rg[j];
    if (SW) su = su + ru[j];
  }
  if (c == 0)
    for (int i = K4; i < K; ++i) {  // the K mod 4 tail into chain 0
      const int64_t item = (int64_t)(n / H) * nb * H + (int64_t)(i >> 5) * H + (n % H);
      sg = sg + sx[i] * (float)*reinterpret_cast<const int8_t*>(tg.data + item * 32 + (i & 31));
      if (SW) su = su + sx[i] * (float)*reinterpret_cast<const int8_t*>(a.tg[1].data + item * 32 + (i & 31));
    }
  const float pg = sg + __shfl_xor(sg, 1);  // lane 4r: s0 + s1, lane 4r + 2: s2 + s3
  const float g = (pg + __shfl_xor(pg, 2)) * tg.scales[n];
  float up = 0.f;
  if (SW) {
    const float pu = su + __shfl_xor(su, 1);
    up = (pu + __shfl_xor(pu, 2)) * a.tg[1].scales[n];
  }
  if (c == 0 && n < tg.N) {
    if (SW) tg.y[n] = silu_exact(g) * up;
    else tg.y[n] = (tg.res ? tg.res[n] : 0.f) + g;
  }
}

// The same with the workgroup's rows first copied into LDS (global_load_lds, all in flight at
// once; one wait): row r of selection sel is its K bytes (32 nb, the layout's block padding
// included) plus one 16-byte pad at LDS byte ((sel * 16 + r) * (2 nb + 1)) * 16, so the 16 rows'
// reads of one step fall on different banks. x follows in LDS. Used while that fits 64 KB.
constexpr int kQ8F32LdsRows = 16;
__host__ __device__ inline int q8f32_chunks(int nb, int nsel) { return nsel * kQ8F32LdsRows * (2 * nb + 1); }
template <bool SW>
__global__ __launch_bounds__(64) void gemv_f32act_q8_lds_kernel(const F32Args a) {
  extern __shared__ __align__(16) unsigned char q8l_lds[];
  constexpr int NSEL = SW ? 2 : 1;
  const int K = a.K, K4 = K & ~3, H = a.H, nb = a.nb, cpr = 2 * nb + 1, lane = threadIdx.x;
  int grp = blockIdx.x;
  const GemvTarget tg = f32_target<SW>(a, grp);
  const int n0 = grp * kQ8F32LdsRows;  // rows past N: padding (rows_pad % 64 == 0)
  const int nch = q8f32_chunks(nb, NSEL);
  unsigned char* const wl = q8l_lds;
  float* const sx = reinterpret_cast<float*>(q8l_lds + ((nch + 63) & ~63) * 16);
  for (int q0 = 0; q0 < nch; q0 += 64) {
    const int q = min(q0 + lane, nch - 1), sel = q / (kQ8F32LdsRows * cpr), rem = q - sel * kQ8F32LdsRows * cpr;
    const int r = rem / cpr, k = min(rem - r * cpr, 2 * nb - 1);  // the pad slot repeats the last chunk
    const int n = n0 + r;
    const int64_t item = (int64_t)(n / H) * nb * H + (int64_t)(k >> 1) * H + (n % H);
    dma16((SW && sel ? a.tg[1].data : tg.data) + item * 32 + (k & 1) * 16, wl + q0 * 16);
  }
  for (int i = lane; i < K; i += 64) sx[i] = a.x[i];
  wait_vm<0>();
  __syncthreads();
  const int c = lane & 3, r = lane >> 2, n = n0 + r;
  const unsigned char* const rg = wl + r * cpr * 16;
  const unsigned char* const ru = wl + (kQ8F32LdsRows + r) * cpr * 16;
  float sg = 0.f, su = 0.f;
  int i = 0;
  for (; i + 16 <= K4; i += 16) {
    const uint4 w = *reinterpret_cast<const uint4*>(rg + i);
    const uint4 wu = SW ? *reinterpret_cast<const uint4*>(ru + i) : w;
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w}, ud[4] = {wu.x, wu.y, wu.z, wu.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float xv = sx[i + 4 * j + c];
      sg = sg + xv * (float)(int8_t)((wd[j] >> (8 * c)) & 0xFF);
      if (SW) su = su + xv * (float)(int8_t)((ud[j] >> (8 * c)) & 0xFF);
    }
  }
  for (; i < K4; i += 4) {
    const float xv = sx[i + c];
    sg = sg + xv * (float)(int8_t)rg[i + c];
    if (SW) su = su + xv * (float)(int8_t)ru[i + c];
  }
  if (c == 0)
    for (; i < K; ++i) {  // the K mod 4 tail into chain 0
      sg = sg + sx[i] * (float)(int8_t)rg[i];
      if (SW) su = su + sx[i] * (float)(int8_t)ru[i];
    }
  const float pg = sg + __shfl_xor(sg, 1);  // lane 0: s0 + s1, lane 2: s2 + s3
  const float g = (pg + __shfl_xor(pg, 2)) * tg.scales[n];
  float up = 0.f;
  if (SW) {
    const float pu = su + __shfl_xor(su, 1);
    up = (pu + __shfl_xor(pu, 2)) * a.tg[1].scales[n];
  }
  if (c == 0 && n < tg.N) {
    if (SW) tg.y[n] = silu_exact(g) * up;
    else tg.y[n] = (tg.res ? tg.res[n] : 0.f) + g;
  }
}

// T == 1, q8: dot_q8's four chains (kernels_cpu.cpp:366-368: chain c takes i = c mod 4 in order,
// the K mod 4 tail goes to chain 0) are independent, so four lanes take one row, a chain each,
// and 16 rows share a one-wave workgroup; the lanes of a row read the same 16 weight bytes and each uses
// its own four. ((s0 + s1) + (s2 + s3)) * ws is formed across the row's lanes.
constexpr int kQ8F32Rows = 16;  // rows per workgroup: one wave, four lanes per row
constexpr int kQ8F32Ahead = 8;  // 16-element steps whose weights are in flight

template <bool SW>
__global__ __launch_bounds__(64) void gemv_f32act_q8_kernel(const F32Args a) {
  extern __shared__ __align__(16) float f32q8_lds[];
  const int K = a.K, K4 = K & ~3, H = a.H;
  int grp = blockIdx.x;
  const GemvTarget tg = f32_target<SW>(a, grp);
  // rows past N: padding (rows_pad % 64 == 0)
  const int c = threadIdx.x & 3, n = grp * kQ8F32Rows + (threadIdx.x >> 2);
  const int64_t nbase = (int64_t)(n / H) * a.nb * H + (n % H);
  const uint8_t* const dg = tg.data;
  const uint8_t* const du = SW ? a.tg[1].data : tg.data;
  const auto at = [&](const uint8_t* d, int i) { return d + (nbase + (int64_t)(i >> 5) * H) * 32 + (i & 31); };
  // the first steps' weights go out before x is staged; each step's weights are loaded
  // kQ8F32Ahead steps before it (gate and up chains side by side with SW)
  const int nst = K4 >> 4;
  uint4 wr[kQ8F32Ahead], ur[kQ8F32Ahead];
#pragma unroll
  for (int u = 0; u < kQ8F32Ahead; ++u)
    if (u < nst) {
      wr[u] = *reinterpret_cast<const uint4*>(at(dg, 16 * u));
      if (SW) ur[u] = *reinterpret_cast<const uint4*>(at(du, 16 * u));
    }
  for (int i = threadIdx.x; i < K; i += 64) f32q8_lds[i] = a.x[i];
  __syncthreads();
  float sg = 0.f, su = 0.f;
  for (int s0 = 0; s0 < nst; s0 += kQ8F32Ahead) {
#pragma unroll
    for (int u = 0; u < kQ8F32Ahead; ++u) {
      const int st = s0 + u, i = 16 * st;
      if (st < nst) {
        const uint4 w = wr[u];
        const uint4 wu = SW ? ur[u] : w;
        if (st + kQ8F32Ahead < nst) {
          wr[u] = *reinterpret_cast<const uint4*>(at(dg, i + 16 * kQ8F32Ahead));
          if (SW) ur[u] = *reinterpret_cast<const uint4*>(at(du, i + 16 * kQ8F32Ahead));
        }
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w}, ud[4] = {wu.x, wu.y, wu.z, wu.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float xv = f32q8_lds[i + 4 * j + c];
          sg = sg + xv * (float)(int8_t)((wd[j] >> (8 * c)) & 0xFF);
          if (SW) su = su + xv * (float)(int8_t)((ud[j] >> (8 * c)) & 0xFF);
        }
      }
    }
  }
  int i = 16 * nst;
  for (; i < K4; i += 4) {
    const float xv = f32q8_lds[i + c];
    sg = sg + xv * (float)(int8_t)((*reinterpret_cast<const uint32_t*>(at(dg, i)) >> (8 * c)) & 0xFF);
    if (SW) su = su + xv * (float)(int8_t)((*reinterpret_cast<const uint32_t*>(at(du, i)) >> (8 * c)) & 0xFF);
  }
  if (c == 0)
    for (; i < K; ++i) {  // the K mod 4 tail into chain 0
      sg = sg + f32q8_lds[i] * (float)*reinterpret_cast<const int8_t*>(at(dg, i));
      if (SW) su = su + f32q8_lds[i] * (float)*reinterpret_cast<const int8_t*>(at(du, i));
    }
  const float pg = sg + __shfl_xor(sg, 1);  // lane 0: s0 + s1, lane 2: s2 + s3
  const float g = (pg + __shfl_xor(pg, 2)) * tg.scales[n];
  float up = 0.f;
  if (SW) {
    const float pu = su + __shfl_xor(su, 1);
    up = (pu + __shfl_xor(pu, 2)) * a.tg[1].scales[n];
  }
  if (c == 0 && n < tg.N) {
    if (SW) tg.y[n] = silu_exact(g) * up;
    else tg.y[n] = (tg.res ? tg.res[n] : 0.f) + g;
  }
}

// T > 1 (kernels_cpu.cpp:369-371, 401-403): the weight tile is dequantized (float(q) * s, one
// rounding) and dotted in dot_f32_scalar's four chains (chain c takes i = c mod 4 in order, the
// K mod 4 tail goes to chain 0); y = (res or 0) + dot. The chains are independent, so four lanes
// take one (row, kF32TT tokens) tile, a chain each: a workgroup is 64 rows x kF32TT tokens (2
// tokens measured faster than 4 or 8 at the 135M model's 128-token prefill, which has too few
// (row, token) pairs to fill the chip with more tokens per lane). x is staged
// through LDS by chain ([token][chain][k / 4], so a lane reads four of its chain's values at
// once), and the row's four lanes read the same 16 weight bytes, each using its own four.
constexpr int kF32TT = 2;
constexpr int kF32Chunk = 2048;
constexpr int kF32ChainStride = kF32Chunk / 4 + 4;  // floats; the +4 spreads the staging writes over banks

template <int WDT>
__device__ __forceinline__ float deq1(const uint8_t* __restrict__ data, const float* __restrict__ scales,
                                      int64_t nbase, int H, int i, int n) {
  const int b = i >> 5;
  const int64_t item = nbase + (int64_t)b * H;
  if (WDT == WQ8) return (float)*reinterpret_cast<const int8_t*>(data + item * 32 + (i & 31)) * scales[n];
  const int e = i & 31;
  const uint8_t byte = data[item * 16 + (e & 15)];
  return (float)((int)(e >= 16 ? byte >> 4 : byte & 0x0F) - 8) * scales[item];
}

// The 16 weight bytes that hold elements i .. i + 15 of row n (i % 16 == 0) and their scale
struct WChunk {
  uint4 q;
  float s;
};
template <int WDT>
__device__ __forceinline__ WChunk load_chunk(const uint8_t* __restrict__ data, const float* __restrict__ scales,
                                             int64_t nbase, int H, int i, int n) {
  const int64_t item = nbase + (int64_t)(i >> 5) * H;
  if (WDT == WQ8) return {*reinterpret_cast<const uint4*>(data + item * 32 + (i & 31)), scales[n]};
  return {*reinterpret_cast<const uint4*>(data + item * 16), scales[item]};  // the group: byte m holds m, m + 16
}
// chain c's four dequantized weights of the chunk: elements i + c + 4m, m = 0 .. 3
template <int WDT>
__device__ __forceinline__ float4 chunk_chain(const WChunk& w, int i, int c) {
  float4 r;
  if (WDT == WQ8) {
    r.x = (float)(int8_t)((w.q.x >> (8 * c)) & 0xFF) * w.s;
    r.y = (float)(int8_t)((w.q.y >> (8 * c)) & 0xFF) * w.s;
    r.z = (float)(int8_t)((w.q.z >> (8 * c)) & 0xFF) * w.s;
    r.w = (float)(int8_t)((w.q.w >> (8 * c)) & 0xFF) * w.s;
  } else {
    const int sh = 8 * c + ((i & 31) >= 16 ? 4 : 0);
    r.x = (float)((int)((w.q.x >> sh) & 0x0F) - 8) * w.s;
    r.y = (float)((int)((w.q.y >> sh) & 0x0F) - 8) * w.s;
    r.z = (float)((int)((w.q.z >> sh) & 0x0F) - 8) * w.s;
    r.w = (float)((int)((w.q.w >> sh) & 0x0F) - 8) * w.s;
  }
  return r;
}
constexpr int kF32Ahead = 4;  // 16-element steps whose weights are in flight

template <int WDT, bool SW>
__global__ __launch_bounds__(256) void gemm_f32act_kernel(const F32Args a) {
  __shared__ __align__(16) float sxp[kF32TT][4][kF32ChainStride];
  int grp = blockIdx.y;
  const GemvTarget tg = f32_target<SW>(a, grp);
  const int K = a.K, K4 = K & ~3, H = a.H, nb = a.nb, T = a.T;
  const int t0 = blockIdx.x * kF32TT, c = threadIdx.x & 3;
  const int n = grp * 64 + (threadIdx.x >> 2);  // rows past N: padding (rows_pad % 64 == 0)
  const int64_t nbase = (int64_t)(n / H) * nb * H + (n % H);
  float s[kF32TT], su[kF32TT];
#pragma unroll
  for (int t = 0; t < kF32TT; ++t) s[t] = su[t] = 0.f;
  for (int k0 = 0; k0 < K4; k0 += kF32Chunk) {
    const int klen = min(kF32Chunk, K4 - k0);
    __syncthreads();
    for (int i = threadIdx.x; i < kF32TT * kF32Chunk; i += 256) {
      const int t = i / kF32Chunk, k = i - t * kF32Chunk;
      if (k < klen) sxp[t][k & 3][k >> 2] = t0 + t < T ? a.x[(int64_t)(t0 + t) * K + k0 + k] : 0.f;
    }
    __syncthreads();
    // the chunk's 16-element steps; each step's weights are loaded kF32Ahead steps before it
    const int nst = klen >> 4;
    WChunk wr[kF32Ahead], ur[kF32Ahead];
#pragma unroll
    for (int u = 0; u < kF32Ahead; ++u)
      if (u < nst) {
        wr[u] = load_chunk<WDT>(tg.data, tg.scales, nbase, H, k0 + 16 * u, n);
        if (SW) ur[u] = load_chunk<WDT>(a.tg[1].data, a.tg[1].scales, nbase, H, k0 + 16 * u, n);
      }
    for (int s0 = 0; s0 < nst; s0 += kF32Ahead) {
#pragma unroll
      for (int u = 0; u < kF32Ahead; ++u) {
        const int st = s0 + u, ii = k0 + 16 * st;
        if (st < nst) {
          const float4 w = chunk_chain<WDT>(wr[u], ii, c);
          const float4 wu = SW ? chunk_chain<WDT>(ur[u], ii, c) : w;
          if (st + kF32Ahead < nst) {
            wr[u] = load_chunk<WDT>(tg.data, tg.scales, nbase, H, ii + 16 * kF32Ahead, n);
            if (SW) ur[u] = load_chunk<WDT>(a.tg[1].data, a.tg[1].scales, nbase, H, ii + 16 * kF32Ahead, n);
          }
#pragma unroll
          for (int t = 0; t < kF32TT; ++t) {
            const float4 xv = *reinterpret_cast<const float4*>(&sxp[t][c][(ii - k0) >> 2]);
            s[t] = s[t] + xv.x * w.x;
            s[t] = s[t] + xv.y * w.y;
            s[t] = s[t] + xv.z * w.z;
            s[t] = s[t] + xv.w * w.w;
            if (SW) {
              su[t] = su[t] + xv.x * wu.x;
              su[t] = su[t] + xv.y * wu.y;
              su[t] = su[t] + xv.z * wu.z;
              su[t] = su[t] + xv.w * wu.w;
            }
          }
        }
      }
    }
    int i = k0 + 16 * nst;
    for (; i < k0 + klen; i += 4) {  // the last chunk's steps past its last 16-element run
      const float w = deq1<WDT>(tg.data, tg.scales, nbase, H, i + c, n);
      const float wu = SW ? deq1<WDT>(a.tg[1].data, a.tg[1].scales, nbase, H, i + c, n) : w;
#pragma unroll
      for (int t = 0; t < kF32TT; ++t) {
        const float xv = sxp[t][c][(i - k0) >> 2];
        s[t] = s[t] + xv * w;
        if (SW) su[t] = su[t] + xv * wu;
      }
    }
  }
  if (c == 0)
    for (int i = K4; i < K; ++i) {  // tail (K % 4) into the first chain
      const float w = deq1<WDT>(tg.data, tg.scales, nbase, H, i, n);
      const float wu = SW ? deq1<WDT>(a.tg[1].data, a.tg[1].scales, nbase, H, i, n) : w;
#pragma unroll
      for (int t = 0; t < kF32TT; ++t) {
        const float xv = t0 + t < T ? a.x[(int64_t)(t0 + t) * K + i] : 0.f;
        s[t] = s[t] + xv * w;
        if (SW) su[t] = su[t] + xv * wu;
      }
    }
#pragma unroll
  for (int t = 0; t < kF32TT; ++t) {
    const float p = s[t] + __shfl_xor(s[t], 1);  // lane 0: s0 + s1, lane 2: s2 + s3
    const float dot = p + __shfl_xor(p, 2);
    float out;
    if (SW) {
      const float pu = su[t] + __shfl_xor(su[t], 1);
      const float g = 0.f + dot;
      const float u = 0.f + (pu + __shfl_xor(pu, 2));
      out = silu_exact(g) * u;
    } else {
      out = (t0 + t < T && tg.res ? tg.res[(int64_t)(t0 + t) * tg.N + n] : 0.f) + dot;
    }
    if (c == 0 && n < tg.N && t0 + t < T) tg.y[(int64_t)(t0 + t) * tg.N + n] = out;
  }
}

__global__ void silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ y,
                                int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    y[i] = silu_exact(g[i]) * u[i];
}

// Test hook: S[t][n][b] (exact int32 block sums) from row-major int8 activations.
__global__ void block_sums_kernel(const uint8_t* __restrict__ data, int dtype, int64_t N, int nb, int H,
                                  const int8_t* __restrict__ xq, int T, int32_t* __restrict__ S) {
  const int64_t total = (int64_t)T * N * nb;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = i % nb, n = (i / nb) % N, t = i / (nb * N);
    const int64_t item = item_index(n, b, nb, H);
    const int8_t* xb = xq + t * (int64_t)nb * 32 + b * 32;
    int s = 0;
    if (dtype == WQ8) {
      const int8_t* w = reinterpret_cast<const int8_t*>(data + item * 32);
      for (int e = 0; e < 32; ++e) s += (int)w[e] * (int)xb[e];
    } else {
      const uint8_t* w = data + item * 16;
      for (int e = 0; e < 16; ++e) s += ((int)(w[e] & 0x0F) - 8) * (int)xb[e] + ((int)(w[e] >> 4) - 8) * (int)xb[e + 16];
    }
    S[i] = s;
  }
}

inline int grid_for(int64_t n, int threads, int cap = 65536) {
  const int64_t g = (n + threads - 1) / threads;
  return (int)(g < 1 ? 1 : (g > cap ? cap : g));
}

}  // namespace

// ---------------------------------------------------------------- launchers

hipError_t launch_repack(const uint8_t* raw, const float* raw_scales, DevWeight& w, hipStream_t s) {
  const int64_t items = w.rows_pad * w.nb;
  repack_kernel<<<grid_for(items, 256), 256, 0, s>>>(raw, raw_scales, w.data, w.scales, w.rows, w.cols, w.nb,
                                                      w.rows_pad, w.H, w.dtype);
  return hipGetLastError();
}

hipError_t launch_act_quant_rows(const float* x, int T, int K, int8_t* xq, float* xd, int32_t* xs, hipStream_t s) {
  const int blocks = T * (K / kBlock);
  act_quant_rows_kernel<<<(blocks + 31) / 32, 256, 0, s>>>(x, T, K, xq, xd, xs);
  return hipGetLastError();
}

hipError_t launch_act_quant_frag(const float* x, int T, int Tpad, int K, int8_t* xq, float* xd, hipStream_t s) {
  const dim3 grid(Tpad / 32, (K / kBlock + 3) / 4);
  act_quant_frag_kernel<<<grid, 256, 0, s>>>(x, T, Tpad, K, xq, xd);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_quant_frag(const float* x, const float* nw, float eps, int T, int Tpad, int K, int8_t* xq,
                                     float* xd, hipStream_t s) {
  if (K % kBlock || K > 2048 || Tpad % kNqTok) return hipErrorInvalidValue;
  const size_t rowlen = (size_t)norm_rowlen(K);
  const size_t lds = (size_t)kNqTok * 4 * rowlen * sizeof(float);
  rmsnorm_quant_frag_kernel<<<Tpad / kNqTok, 256, lds, s>>>(x, nw, eps, T, Tpad, K, xq, xd);
  return hipGetLastError();
}

hipError_t launch_act_quant_frag_token(const float* x, int T, int Tpad, int K, int8_t* xq, float* xd, hipStream_t s) {
  const int k4 = K / 4;  // float4s per row
  if (k4 <= 256)
    act_quant_frag_token_kernel<1><<<Tpad, 256, 0, s>>>(x, T, Tpad, K, xq, xd);
  else if (k4 <= 1024)
    act_quant_frag_token_kernel<4><<<Tpad, 256, 0, s>>>(x, T, Tpad, K, xq, xd);
  else if (k4 <= 4096)
    act_quant_frag_token_kernel<16><<<Tpad, 256, 0, s>>>(x, T, Tpad, K, xq, xd);
  else
    act_quant_frag_token_kernel<0><<<Tpad, 256, 0, s>>>(x, T, Tpad, K, xq, xd);
  return hipGetLastError();
}

int gemv_max_tokens(int K) {
  if (K <= 4096) return 4;
  if (K <= 8192) return 2;
  if (K <= 16384) return 1;
  return 0;
}

size_t gemv_lds_bytes(int nt, int K, int nb, int H, int nsel) {
  const size_t kpad = (size_t)((K + 15) & ~15);
  const size_t p = (size_t)((nb + 3) & ~3);
  const size_t pst = ((p >> 2) & 1) ? p : p + 4;
  return nt * kpad + (((size_t)nt * nb * 8 + 15) & ~(size_t)15) + (size_t)nsel * nt * H * pst * 4;
}

bool gemv_qin_ok(int T, int K) { return T * K <= kSmallMaxAct; }

int gemv_stream_ipt(int dtype, int items, int producers) {
  const int per = (items + producers - 1) / producers;
  const int cap = dtype == WQ8 ? 8 : 16;
  if (per > cap) return 0;
  return per <= 4 ? 4 : per <= 8 ? 8 : 16;
}

// MT: the launch has more than one target (a fused QKV); only such launches look the target up.
template <int WDT, int NT, bool SW, int NPW, bool FW, bool QIN, bool QOUT, bool MT>
static hipError_t stream_launch_mt(const GemvArgs& a, int wgs, size_t lds, int items, hipStream_t s) {
  constexpr int threads = 64 * (NPW + FW);
  switch (gemv_stream_ipt(WDT, items, 64 * NPW)) {
    case 4: gemv_stream_kernel<WDT, NT, SW, 4, NPW, FW ? 2 : 4, FW, QIN, QOUT, MT><<<wgs, threads, lds, s>>>(a); break;
    case 8: gemv_stream_kernel<WDT, NT, SW, 8, NPW, FW ? 2 : 4, FW, QIN, QOUT, MT><<<wgs, threads, lds, s>>>(a); break;
    case 16:
      if (WDT == WQ4) {
        gemv_stream_kernel<WDT, NT, SW, 16, NPW, FW ? 2 : 4, FW, QIN, QOUT, MT><<<wgs, threads, lds, s>>>(a);
        break;
      }
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int WDT, int NT, bool SW, int NPW, bool FW, bool QIN, bool QOUT = false>
static hipError_t stream_launch(const GemvArgs& a, int wgs, size_t lds, int items, hipStream_t s) {
  if constexpr (!SW) {
    if (a.n_targets > 1) return stream_launch_mt<WDT, NT, false, NPW, FW, QIN, QOUT, true>(a, wgs, lds, items, s);
  }
  return stream_launch_mt<WDT, NT, SW, NPW, FW, QIN, QOUT, false>(a, wgs, lds, items, s);
}

template <int WDT, int NT, bool SW, int NPW, bool FW>
static hipError_t stream_go(const GemvArgs& a, int wgs, size_t lds, int items, hipStream_t s) {
  if (a.x) return stream_launch<WDT, NT, SW, NPW, FW, true>(a, wgs, lds, items, s);
  return stream_launch<WDT, NT, SW, NPW, FW, false>(a, wgs, lds, items, s);
}

template <int WDT, int NT, bool SW>
static hipError_t gemv_go(const GemvArgs& a, int tiles, hipStream_t s) {
  if (a.T > NT) return hipErrorInvalidValue;
  const int rs = a.rsub ? a.rsub : a.H;  // small kernel: rows per workgroup
  const size_t lds = gemv_lds_bytes(NT, a.K, a.nb, a.x && !a.stream ? rs : a.tpw * a.H, SW ? 2 : 1);
  if (lds > 64 * 1024) return hipErrorInvalidValue;
  if (a.x && !a.stream) {
    if (!gemv_qin_ok(a.T, a.K) || (a.K & 31) || (a.H & (a.H - 1)) || (rs & (rs - 1)) || rs > a.H ||
        a.T * rs * (SW ? 2 : 1) > kGemvThreads)
      return hipErrorInvalidValue;
    if (a.nw) {
      const size_t rowlen = (size_t)norm_rowlen(a.K);
      const size_t ldsn = lds + ((size_t)NT * 4 * rowlen + 4) * sizeof(float);
      if (ldsn > 64 * 1024) return hipErrorInvalidValue;
      if constexpr (!SW) {
        if (a.n_targets > 1) {
          gemv_small_kernel<WDT, NT, false, true, true><<<tiles, kGemvThreads, ldsn, s>>>(a);
          return hipGetLastError();
        }
      }
      gemv_small_kernel<WDT, NT, SW, true, false><<<tiles, kGemvThreads, ldsn, s>>>(a);
    } else {
      if constexpr (!SW) {
        if (a.n_targets > 1) {
          gemv_small_kernel<WDT, NT, false, false, true><<<tiles, kGemvThreads, lds, s>>>(a);
          return hipGetLastError();
        }
      }
      gemv_small_kernel<WDT, NT, SW, false, false><<<tiles, kGemvThreads, lds, s>>>(a);
    }
    return hipGetLastError();
  }
  if (a.tpw < 1 || a.T * a.tpw * a.H > kStreamFoldLanes || a.T * a.K > kStreamMaxAct || (a.K & 15) ||
      (a.H & (a.H - 1)) || a.H > 64 || a.tpw * a.nb > 4096 || (a.x && !stream_qin_ok(a.T, a.K)) || a.nw)
    return hipErrorInvalidValue;
  if (SW && a.T == 1 && a.x && a.tpw * a.H == 32) {
    // SwiGLU, one token, x quantized per workgroup, short rows (the fold at the end): 32-row
    // workgroups of kStreamQoutWaves producer waves, the output row also quantized in the fold when
    // oq is set
    if constexpr (SW && NT == 1) {
      if (a.nb > kStreamFoldWaveBlocks || (a.oq && (!a.od || !a.os || (a.tg[0].N & 31)))) return hipErrorInvalidValue;
      return stream_launch<WDT, 1, true, kStreamQoutWaves, false, true, true>(a, tiles, lds, 2 * 32 * a.nb, s);
    } else {
      return hipErrorInvalidValue;
    }
  }
  const int items = (SW ? 2 : 1) * a.tpw * a.H * a.nb;
  if (a.nb > kStreamFoldWaveBlocks) return stream_go<WDT, NT, SW, kStreamWavesLong, true>(a, tiles, lds, items, s);
  return stream_go<WDT, NT, SW, kStreamWavesShort, false>(a, tiles, lds, items, s);
}

template <int WDT, bool SW>
static hipError_t gemv_nt(const GemvArgs& a, int tiles, hipStream_t s) {
  if (a.T <= 1) return gemv_go<WDT, 1, SW>(a, tiles, s);
  if (a.T <= 2) return gemv_go<WDT, 2, SW>(a, tiles, s);
  return gemv_go<WDT, 4, SW>(a, tiles, s);
}

hipError_t launch_gemv_a8(int dtype, int swiglu, const GemvArgs& a, int total_tiles, hipStream_t s) {
  if (a.T > 4) return hipErrorInvalidValue;
  if (dtype == WQ8) return swiglu ? gemv_nt<WQ8, true>(a, total_tiles, s) : gemv_nt<WQ8, false>(a, total_tiles, s);
  return swiglu ? gemv_nt<WQ4, true>(a, total_tiles, s) : gemv_nt<WQ4, false>(a, total_tiles, s);
}

template <int WDT, bool SW, bool TOK, int MT, int WV = 4>
static void gemm_launch(const GemmArgs& a, dim3 grid, hipStream_t s) {
  // edgelm's per-block mode, 64-token tiles: one barrier per group of six blocks. Measured at T = 512
  // against one per block: q8 4096 x 4096 47.7 -> 45.6 us, 4096 x 14336 126.1 -> 117.8 us, 14336 x
  // 4096 95.0 -> 95.9 us (four blocks per group 46.3 / 121.1 / 96.5 us, two 51.3 / 144.6 / 98.4 us);
  // q4 against its block-pipelined eight-wave loop 58.4 -> 56.7, 161.5 -> 154.8, 117.5 -> 117.6 us.
  // ELMH_GEMM_KB=1 keeps one barrier per block (q4: the pipelined loop); same bits.
  if constexpr (!SW && !TOK && MT == 1) {
    const char* ev = getenv("ELMH_GEMM_KB");
    if (!(ev && ev[0] == '1')) {
      if (a.fast)
        gemm_a8_kernel<WDT, SW, TOK, true, MT, 6, WV><<<grid, 64 * WV, 0, s>>>(a);
      else
        gemm_a8_kernel<WDT, SW, TOK, false, MT, 6, WV><<<grid, 64 * WV, 0, s>>>(a);
      return;
    }
  }
  // the per-token q8 accumulation is all-integer: FAST changes nothing there
  if (a.fast && !(TOK && WDT == WQ8))
    gemm_a8_kernel<WDT, SW, TOK, true, MT, 0, WV><<<grid, 64 * WV, 0, s>>>(a);
  else
    gemm_a8_kernel<WDT, SW, TOK, false, MT, 0, WV><<<grid, 64 * WV, 0, s>>>(a);
}

// The ring GEMM with four or eight waves (eight: without SwiGLU; q8 in the block-scale mode where the
// grid gives at most one workgroup per CU, so that four waves would leave one wave per SIMD, q4
// always; per-token q8, whose loop is all MFMA, measured slower with eight: 26.4 -> 28.4 us at
// 4096 x 4096, 61.8 -> 65.4 us at 4096 x 14336, while per-token q4 gained: 63.8 -> 51.5, 99.7 -> 97.8,
// 189.7 -> 140.1 us).
// Measured at T = 512: q8 4096 x 4096 59.2 -> 48.3 us, 4096 x 14336 173.4 -> 133.4 us, while 14336 x
// 4096 with 448 workgroups went from 98.8 to 103.7 us; q4 (pipelined eight-wave loop) 78.0 -> 60.6,
// 228.7 -> 160.7 and, at 448 workgroups, 125.8 -> 120.2 us. ELMH_GEMM_WAVES=4 or 8 forces one, same
// bits.
template <int WDT, bool SW, bool TOK, int MT>
static void gemm_launch_waves(const GemmArgs& a, int wgs, int cus, hipStream_t s) {
  const dim3 grid((wgs + 7) / 8 * 8);
  if constexpr (!SW) {
    bool eight = WDT == WQ4 || (!TOK && wgs <= cus);
    if (const char* ev = getenv("ELMH_GEMM_WAVES")) eight = ev[0] == '8' ? true : ev[0] == '4' ? false : eight;
    if (eight) return gemm_launch<WDT, SW, TOK, MT, 8>(a, grid, s);
  }
  gemm_launch<WDT, SW, TOK, MT>(a, grid, s);
}

template <int WDT, bool SW, bool TOK>
static void gemm_wave_launch(const GemmArgs& a, hipStream_t s) {
  int rows = 0;
  for (int i = 0; i < (SW ? 1 : a.n_targets); ++i) rows += (a.tg[i].N + kWaveTile - 1) / kWaveTile;
  const int waves = rows * ((a.T + kWaveTile - 1) / kWaveTile);
  const dim3 grid((waves + 3) / 4);
  if (a.fast && !(TOK && WDT == WQ8))
    gemm_wave_kernel<WDT, SW, TOK, true><<<grid, 256, 0, s>>>(a);
  else
    gemm_wave_kernel<WDT, SW, TOK, false><<<grid, 256, 0, s>>>(a);
}

template <int WDT, bool SW, bool TOK>
static void gemm_wave16_launch(const GemmArgs& a, hipStream_t s) {
  int rows = 0;
  for (int i = 0; i < (SW ? 1 : a.n_targets); ++i) rows += (a.tg[i].N + kWave16 - 1) / kWave16;
  const int waves = rows * ((a.T + kWave16 - 1) / kWave16);
  const dim3 grid((waves + 3) / 4);
  if (a.fast && !(TOK && WDT == WQ8))
    gemm_wave16_kernel<WDT, SW, TOK, true><<<grid, 256, 0, s>>>(a);
  else
    gemm_wave16_kernel<WDT, SW, TOK, false><<<grid, 256, 0, s>>>(a);
}

// gemm_lds16_kernel when its LDS fits (K <= 1536 or so); false otherwise
template <int WDT, bool SW, bool TOK, bool QF = false>
static bool gemm_lds16_launch(const GemmArgs& a, hipStream_t s) {
  const int bytes = gemm_lds16_bytes<WDT, SW, TOK, QF>(a.nb);
  if (a.nb > kLds16MaxBlocks || bytes > (int)kMaxLds - 1024 || a.H < 4 || (a.H & (a.H - 1))) return false;
  const bool fast = a.fast && !(TOK && WDT == WQ8), mt = !SW && a.n_targets > 1;
  // the kernel for (fast, more than one target); SwiGLU has one
  const void* const ks[4] = {(const void*)gemm_lds16_kernel<WDT, SW, TOK, false, QF, false>,
                             (const void*)gemm_lds16_kernel<WDT, SW, TOK, true, QF, false>,
                             (const void*)gemm_lds16_kernel<WDT, SW, TOK, false, QF, !SW>,
                             (const void*)gemm_lds16_kernel<WDT, SW, TOK, true, QF, !SW>};
  static bool raised[4] = {false, false, false, false};  // the LDS limit, once per kernel
  const int which = (mt ? 2 : 0) + (fast ? 1 : 0);
  if (!raised[which]) {
    if (hipFuncSetAttribute(ks[which], hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds - 1024) != hipSuccess)
      return false;
    raised[which] = true;
  }
  constexpr int RW = QF ? 32 : 16, TW = QF ? 32 : 64;
  int rows = 0;
  for (int i = 0; i < (SW ? 1 : a.n_targets); ++i) rows += (a.tg[i].N + RW - 1) / RW;
  const dim3 grid(rows * ((a.T + TW - 1) / TW));
  switch (which) {
    case 0: gemm_lds16_kernel<WDT, SW, TOK, false, QF, false><<<grid, 256, bytes, s>>>(a); break;
    case 1: gemm_lds16_kernel<WDT, SW, TOK, true, QF, false><<<grid, 256, bytes, s>>>(a); break;
    case 2: gemm_lds16_kernel<WDT, SW, TOK, false, QF, !SW><<<grid, 256, bytes, s>>>(a); break;
    default: gemm_lds16_kernel<WDT, SW, TOK, true, QF, !SW><<<grid, 256, bytes, s>>>(a); break;
  }
  return true;
}

// Whether a SwiGLU GEMM in block mode can write h's quantized fragments itself (gemm_lds16_kernel's
// 32 x 32 workgroups): where the 16 x 16 wave kernels would run it anyway (few token tiles) and
// their LDS holds it, N a multiple of 32
bool gemm_qf_ok(int dtype, int T, int nb, int H, int N, int64_t rows_pad) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return false;
  const int tiles = (int)((rows_pad + kGemmTileN - 1) / kGemmTileN);
  const int bytes = dtype == WQ8 ? gemm_lds16_bytes<WQ8, true, false, true>(nb) : gemm_lds16_bytes<WQ4, true, false, true>(nb);
  return tiles * ((T + 63) / 64) < cus / 2 && nb <= kLds16MaxBlocks && bytes <= (int)kMaxLds - 1024 && H >= 4 &&
         !(H & (H - 1)) && N % kBlock == 0 && !getenv("ELMH_GEMM_KERNEL") && !getenv("ELMH_GEMM_TOKEN_TILE");
}

template <int WDT, bool SW, bool TOK>
static hipError_t gemm_go(const GemmArgs& a, int tiles, hipStream_t s) {
  if (a.Tpad % kGemmTileT || a.T < 1 || a.T > a.Tpad || tiles < 1 ||
      tiles != (SW ? a.tg[0].ntiles : a.tile_start[a.n_targets]))
    return hipErrorInvalidValue;
  // the epilogue's buffer resources span 128 tokens x N floats in 31 bits
  for (int i = 0; i < (SW ? 2 : a.n_targets); ++i)
    if (a.tg[i].N < 1 || a.tg[i].N >= (1 << 22)) return hipErrorInvalidValue;
  if (a.oq) {  // h's quantized fragments out of the SwiGLU GEMM (gemm_qf_ok holds)
    if constexpr (SW && !TOK) {
      if (!a.od || a.tg[0].N % kBlock || a.onb != a.tg[0].N / kBlock) return hipErrorInvalidValue;
      return gemm_lds16_launch<WDT, SW, TOK, true>(a, s) ? hipGetLastError() : hipErrorInvalidValue;
    } else {
      return hipErrorInvalidValue;
    }
  }
  // one workgroup per (row tile, token tile), numbered in 8 XCD-contiguous ranges; 64-token tiles
  // when 128-token tiles would leave compute units idle
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  // token tiles are counted from T, so every tile starts at a valid token (its store range is
  // min(TT, T - t0) >= 1 tokens)
  const int t128 = tiles * ((a.T + 127) / 128), t64 = tiles * ((a.T + 63) / 64);
  // per-token q8 keeps 128-token tiles down to half the CUs: its loop is all MFMA, and two token
  // groups per wave gained more than the idle CUs cost (T = 512: 4096 x 4096 26.4 -> 25.6 us,
  // 4096 x 14336 62.3 -> 57.8 us; the per-block modes lost: 44.2 -> 61.6, 110.7 -> 183.4 us)
  bool small = TOK && WDT == WQ8 && !SW ? t128 < cus / 2 : t128 < cus;
  // problems that give the ring kernel fewer workgroups than half the CUs: one wave per 32 x 32 tile
  bool wave = t64 < cus / 2;
  // ELMH_GEMM_TOKEN_TILE=64 or 128 forces the ring kernel with one tile height; ELMH_GEMM_KERNEL=wave
  // or ring forces the kernel (all give the same bits)
  if (const char* ev = getenv("ELMH_GEMM_TOKEN_TILE")) {
    small = ev[0] == '6' ? true : ev[0] == '1' ? false : small;
    wave = false;
  }
  // 16 x 16 waves with their operands staged in LDS (gemm_lds16_kernel) where they fit, else
  // loaded from L2 (gemm_wave16_kernel); ELMH_GEMM_KERNEL = lds16, wave (16 x 16 from L2), wave32
  // or ring forces a kernel
  bool wave32 = false, lds16 = true;
  if (const char* ev = getenv("ELMH_GEMM_KERNEL")) {
    wave = ev[0] == 'w' || ev[0] == 'l' ? true : ev[0] == 'r' ? false : wave;
    wave32 = std::strcmp(ev, "wave32") == 0;
    lds16 = ev[0] == 'l';
  }
  if (wave) {
    if (wave32)
      gemm_wave_launch<WDT, SW, TOK>(a, s);
    else if (!lds16 || !gemm_lds16_launch<WDT, SW, TOK>(a, s))
      gemm_wave16_launch<WDT, SW, TOK>(a, s);
    return hipGetLastError();
  }
  if (small)
    gemm_launch_waves<WDT, SW, TOK, 1>(a, t64, cus, s);
  else
    gemm_launch_waves<WDT, SW, TOK, 2>(a, t128, cus, s);
  return hipGetLastError();
}
hipError_t launch_gemm_a8(int dtype, int swiglu, int token_mode, const GemmArgs& a, int total_tiles, hipStream_t s) {
  // the ring GEMM addresses its DMA sources as a scalar base plus a 32-bit lane offset
  const int64_t G = dtype == WQ8 ? 32 : 16, lim = int64_t(1) << 31;
  if ((int64_t)a.Tpad * a.K >= lim) return hipErrorInvalidValue;
  for (int i = 0; i < (swiglu ? 2 : a.n_targets); ++i)
    if ((a.tg[i].N + kPadRows - 1) / kPadRows * (int64_t)kPadRows * a.nb * G >= lim) return hipErrorInvalidValue;
  if (dtype == WQ8) {
    if (token_mode) return swiglu ? gemm_go<WQ8, true, true>(a, total_tiles, s) : gemm_go<WQ8, false, true>(a, total_tiles, s);
    return swiglu ? gemm_go<WQ8, true, false>(a, total_tiles, s) : gemm_go<WQ8, false, false>(a, total_tiles, s);
  }
  if (token_mode) return swiglu ? gemm_go<WQ4, true, true>(a, total_tiles, s) : gemm_go<WQ4, false, true>(a, total_tiles, s);
  return swiglu ? gemm_go<WQ4, true, false>(a, total_tiles, s) : gemm_go<WQ4, false, false>(a, total_tiles, s);
}

// LDS of gemv_f32act_q4_kernel: x, the (selection, row, group) products and, with RMSNORM, the squares
static size_t f32q4_lds_bytes(int K, int nb, int H, int nsel, bool norm) {
  const size_t base = ((size_t)((K + 3) & ~3) + (size_t)nsel * H * (nb + 1) + 3) & ~(size_t)3;
  return (base + (norm ? 4 * (size_t)norm_rowlen(K) : 0)) * sizeof(float);
}

// Rows per workgroup of gemv_f32act_q4_kernel (a divisor of H): the most rows whose (selection, row,
// group) items take one pass of the 256 threads, raised while that makes more than 1024 workgroups
// (each one stages all of x). rows: the output rows of the call.
static int f32q4_tile_rows(int H, int nb, int nsel, int rows) {
  int rt = H;
  while (rt > 1 && nsel * rt * nb > 256) rt >>= 1;
  while (rt < H && (rows + rt - 1) / rt > 1024) rt <<= 1;
  return rt;
}

bool f32act_q4_ok(int T, int K, int nb, int H, int nsel, int rows, bool norm) {
  return T == 1 && H >= 1 && !(H & (H - 1)) && K == nb * kBlock &&
         f32q4_lds_bytes(K, nb, f32q4_tile_rows(H, nb, nsel, rows), nsel, norm) <= kMaxLds - 1024;
}

hipError_t launch_f32act(int dtype, int swiglu, const F32Args& a, hipStream_t s) {
  const int nsel = swiglu ? 2 : 1;
  const int n = swiglu ? 1 : a.n_targets;
  int rows = 0;
  for (int i = 0; i < n; ++i) rows += a.tg[i].N;
  if (a.T == 1 && dtype == WQ4 && f32act_q4_ok(a.T, a.K, a.nb, a.H, nsel, rows, a.nw != nullptr)) {
    // one workgroup per tile of rt rows; the tile starts counted in tiles here
    F32Args b = a;
    const int rt = f32q4_tile_rows(a.H, a.nb, nsel, rows);
    b.rt = rt;
    int tiles = 0;
    for (int i = 0; i < n; ++i) {
      b.tile_start[i] = tiles;
      tiles += (a.tg[i].N + rt - 1) / rt;
    }
    b.tile_start[n] = tiles;
    const size_t lds = f32q4_lds_bytes(a.K, a.nb, rt, nsel, a.nw != nullptr);
    if (tiles < 1) return hipErrorInvalidValue;
    static bool raised[2] = {false, false};  // the LDS limit, once per kernel
    if (lds > 64 * 1024 && !raised[nsel - 1]) {
      const void* k = swiglu ? (const void*)gemv_f32act_q4_kernel<true> : (const void*)gemv_f32act_q4_kernel<false>;
      const hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds - 1024);
      if (e != hipSuccess) return e;
      raised[nsel - 1] = true;
    }
    if (swiglu) gemv_f32act_q4_kernel<true><<<tiles, 256, lds, s>>>(b);
    else gemv_f32act_q4_kernel<false><<<tiles, 256, lds, s>>>(b);
    return hipGetLastError();
  }
  if (a.nw) return hipErrorInvalidValue;  // RMSNORM is applied by the q4 GEMV above only
  if (a.T == 1) {
    // q4 always takes the GEMV above (K = 32 nb, H a power of two) unless its LDS would not fit
    if (dtype != WQ8) return hipErrorInvalidValue;
    const size_t lds = (size_t)((a.K + 3) & ~3) * 4;
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    const size_t lds_p = ((size_t)((a.K + 3) & ~3) + (size_t)nsel * kQ8PRows * 4 * q8p_stride(a.K)) * 4;
    // products in LDS while the chains are the bottleneck (a layer's few rows); with many rows (an
    // LM head) the chip is full either way and the four-lane kernels below do less work per row
    if (lds_p <= 64 * 1024 && rows <= 8192) {  // group starts counted in kQ8PRows-row groups here
      F32Args b = a;
      int groups = 0;
      for (int i = 0; i < n; ++i) {
        b.tile_start[i] = groups;
        groups += (a.tg[i].N + kQ8PRows - 1) / kQ8PRows;
      }
      b.tile_start[n] = groups;
      if (groups < 1) return hipErrorInvalidValue;
      if (swiglu) gemv_f32act_q8_prod_kernel<true><<<groups, 256, lds_p, s>>>(b);
      else gemv_f32act_q8_prod_kernel<false><<<groups, 256, lds_p, s>>>(b);
      return hipGetLastError();
    }
    // four lanes per row, kQ8F32Rows rows per workgroup; the group starts counted in those here
    F32Args b = a;
    int groups = 0;
    for (int i = 0; i < n; ++i) {
      b.tile_start[i] = groups;
      groups += (a.tg[i].N + kQ8F32Rows - 1) / kQ8F32Rows;
    }
    b.tile_start[n] = groups;
    if (groups < 1) return hipErrorInvalidValue;
    static_assert(kQ8F32Rows == kQ8F32LdsRows, "one grid for both q8 GEMVs");
    const size_t lds_w = (size_t)((q8f32_chunks(a.nb, nsel) + 63) & ~63) * 16 + lds;
    if (lds_w <= 64 * 1024) {
      if (swiglu) gemv_f32act_q8_lds_kernel<true><<<groups, 64, lds_w, s>>>(b);
      else gemv_f32act_q8_lds_kernel<false><<<groups, 64, lds_w, s>>>(b);
    } else if (swiglu) {
      gemv_f32act_q8_kernel<true><<<groups, 64, lds, s>>>(b);
    } else {
      gemv_f32act_q8_kernel<false><<<groups, 64, lds, s>>>(b);
    }
  } else {
    // grid x: kF32TT-token tiles (consecutive workgroups share their weight rows), y: 64-row groups
    F32Args b = a;
    int groups = 0;
    for (int i = 0; i < n; ++i) {
      b.tile_start[i] = groups;
      groups += (a.tg[i].N + 63) / 64;
    }
    b.tile_start[n] = groups;
    if (groups < 1 || groups > 65535) return hipErrorInvalidValue;
    const dim3 grid((a.T + kF32TT - 1) / kF32TT, groups);
    if (dtype == WQ8) {
      if (swiglu) gemm_f32act_kernel<WQ8, true><<<grid, 256, 0, s>>>(b);
      else gemm_f32act_kernel<WQ8, false><<<grid, 256, 0, s>>>(b);
    } else {
      if (swiglu) gemm_f32act_kernel<WQ4, true><<<grid, 256, 0, s>>>(b);
      else gemm_f32act_kernel<WQ4, false><<<grid, 256, 0, s>>>(b);
    }
  }
  return hipGetLastError();
}

hipError_t launch_silu_mul(const float* g, const float* u, float* y, int64_t n, hipStream_t s) {
  silu_mul_kernel<<<grid_for(n, 256), 256, 0, s>>>(g, u, y, n);
  return hipGetLastError();
}

// ---------------------------------------------------------------- rescale ceiling (measurement)

// The per-32-block exact rescale's ceiling on the matrix and vector pipes alone, with no memory
// traffic: each wave runs `iters` steps of two v_mfma_i32_32x32x32_i8 (one 32-deep block of two 32 x 32
// output tiles, as a wave of the ring GEMM does per block; operands in registers, made opaque to the
// compiler each step) and, by MODE, the rescale of the 2 x 16 int32 sums per lane that the per-block
// GEMM does: 0 none (the sums accumulate in the MFMA: the per-token form), 1 q8
// (acc = acc + float(S) * xd, multiply and add rounded separately), 2 q4 (acc = acc + float(S) * (c * xd),
// c the block's weight scale, new every block). Each thread writes one value to sink so that nothing is
// dropped.
template <int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void rescale_ceiling_kernel(int iters,
                                                                                           float* __restrict__ sink) {
  const int tid = threadIdx.x, lane = tid & 63;
  v4i A = {lane, 3 * lane + 1, 5 * lane + 2, 7 * lane + 3};
  v4i B0 = {lane ^ 5, lane + 9, 2 * lane + 7, lane * 11}, B1 = {lane + 1, lane ^ 3, 3 * lane, lane * 13};
  v16i zero;
#pragma unroll
  for (int i = 0; i < 16; ++i) zero[i] = 0;
  float xv[16], f0[16], f1[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    xv[i] = 1.0f / (float)(lane + i + 1);
    f0[i] = f1[i] = 0.f;
  }
  float c0 = 0.25f + 0.001f * (float)lane, c1 = 0.5f - 0.001f * (float)lane;
  v16i acc0 = zero, acc1 = zero;
  for (int k = 0; k < iters; ++k) {
    asm volatile("" : "+v"(A), "+v"(B0), "+v"(B1));  // new operands every block, as far as the compiler knows
    if (MODE == 0) {
      acc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B0, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B1, acc1, 0, 0, 0);
    } else {
      const v16i S0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B0, zero, 0, 0, 0);
      const v16i S1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B1, zero, 0, 0, 0);
      if (MODE == 2) asm volatile("" : "+v"(c0), "+v"(c1));  // the block's weight scales
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        f0[i] = f0[i] + (float)S0[i] * (MODE == 1 ? xv[i] : c0 * xv[i]);
        f1[i] = f1[i] + (float)S1[i] * (MODE == 1 ? xv[i] : c1 * xv[i]);
      }
    }
  }
  float out = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) out = out + (MODE == 0 ? (float)(acc0[i] ^ acc1[i]) : f0[i] + f1[i]);
  sink[(size_t)blockIdx.x * blockDim.x + tid] = out;
}

hipError_t launch_rescale_ceiling(int mode, int blocks, int iters, float* sink, hipStream_t s) {
  if (mode == 0) rescale_ceiling_kernel<0><<<blocks, 256, 0, s>>>(iters, sink);
  else if (mode == 1) rescale_ceiling_kernel<1><<<blocks, 256, 0, s>>>(iters, sink);
  else rescale_ceiling_kernel<2><<<blocks, 256, 0, s>>>(iters, sink);
  return hipGetLastError();
}

hipError_t launch_block_sums(const DevWeight& w, const int8_t* xq, int T, int32_t* S, hipStream_t s) {
  block_sums_kernel<<<grid_for((int64_t)T * w.rows * w.nb, 256), 256, 0, s>>>(w.data, w.dtype, w.rows, (int)w.nb, w.H,
                                                                              xq, T, S);
  return hipGetLastError();
}

}  // namespace elmh

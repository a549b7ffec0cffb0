// The non-matmul ops of a transformer layer on the device, so that a whole layer stays in HBM
// between consecutive ops: token embedding, RMSNORM, and attention with the rotary embedding and
// the KV-cache append fused in. Every float operation happens in the order of edgelm's cpu
// backend (x86 scalar path, no FMA contraction), so results are bit-identical to it:
//   rmsnorm   kernels_cpu.cpp:326-335 with dot_f32_scalar (kernels_cpu.cpp:30-43)
//   attention kernels_cpu.cpp:417-488 (append with rotated keys, then one task per (token, head))
//   embed     dequantize_row (model.cpp:192-218) of the token's row, EMBED (backends.cpp, reference)
#include <hip/hip_runtime.h>

#include "elm_dma.h"
#include "elm_dpp.h"
#include "elm_expf.h"
#include "elm_quant.h"
#include "elm_sum.h"
#include "elmh_internal.hpp"

namespace elmh {
namespace {

// four floats as one vector value: copies stay register moves (a float4 struct copy between
// memory spaces can become a memcpy that keeps an array of them out of registers)
typedef float v4f __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- RMSNORM
//
// One workgroup per row: dot_f32_scalar's four strided accumulators s_k = sum of x[i]^2 over
// i = k (mod 4) in increasing i (the tail past the last multiple of 4 goes into s0), then
// ss = (s0 + s1) + (s2 + s3); inv = 1 / sqrt(ss / dim + eps); y[i] = (x[i] * inv) * w[i].
// Every thread squares its float4s (the products are separate roundings in the scalar code too)
// and writes them to LDS by accumulator: row k holds the terms of s_k in order, zero-padded to a
// multiple of 32 (adding +0.0 to a sum of squares, which is never -0.0, changes nothing). Lanes
// 0-3 then run the four sums, reading eight float4 before their 32 dependent adds, and combine
// them with two DPP steps. x and w stay in registers for the output.
constexpr int kNormVF = 8;  // float4 of the row per thread: dim <= 8192

__device__ __forceinline__ float4 ld4u(const float* p) {  // 4-byte aligned is enough
  return make_float4(p[0], p[1], p[2], p[3]);
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                      float* __restrict__ y, int dim, float eps) {
  extern __shared__ float sq[];  // [4][rowlen], then the dim % 4 tail squares
  __shared__ float inv_s;
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x, nq = dim >> 2, rowlen = (nq + 31) & ~31, tail = dim & 3;
  const float* xr = x + r * dim;
  float4 xv[kNormVF], wv[kNormVF];
#pragma unroll
  for (int u = 0; u < kNormVF; ++u) {
    const int i4 = tid + 256 * u;
    if (i4 < nq) {
      xv[u] = ld4u(xr + 4 * i4);
      wv[u] = ld4u(w + 4 * i4);
    }
  }
#pragma unroll
  for (int u = 0; u < kNormVF; ++u) {
    const int i4 = tid + 256 * u;
    if (i4 < rowlen) {
      const bool in = i4 < nq;
      sq[i4] = in ? xv[u].x * xv[u].x : 0.f;
      sq[rowlen + i4] = in ? xv[u].y * xv[u].y : 0.f;
      sq[2 * rowlen + i4] = in ? xv[u].z * xv[u].z : 0.f;
      sq[3 * rowlen + i4] = in ? xv[u].w * xv[u].w : 0.f;
    }
  }
  if (tid < tail) {
    const float v = xr[4 * nq + tid];
    sq[4 * rowlen + tid] = v * v;
  }
  __syncthreads();
  if (tid < 4) {
    const float4* row = reinterpret_cast<const float4*>(sq + tid * rowlen);
    float s = 0.f;
    for (int q0 = 0; q0 < (rowlen >> 2); q0 += 8) {
      float4 v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = row[q0 + i];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        s = s + v[i].x;
        s = s + v[i].y;
        s = s + v[i].z;
        s = s + v[i].w;
      }
    }
    if (tid == 0)
      for (int t = 0; t < tail; ++t) s = s + sq[4 * rowlen + t];
    // lanes 0-3 hold s0..s3: lane 0 forms s0 + s1 and lane 2 s2 + s3, then lane 0 their sum
    const float s01 = s + dpp_f<kDppQuadXor1>(s);
    const float ss = s01 + dpp_f<kDppQuadXor2>(s01);
    if (tid == 0) inv_s = 1.0f / sqrtf(ss / (float)dim + eps);
  }
  __syncthreads();
  const float inv = inv_s;
  float* yr = y + r * dim;
#pragma unroll
  for (int u = 0; u < kNormVF; ++u) {
    const int i4 = tid + 256 * u;
    if (i4 < nq) {
      yr[4 * i4] = (xv[u].x * inv) * wv[u].x;
      yr[4 * i4 + 1] = (xv[u].y * inv) * wv[u].y;
      yr[4 * i4 + 2] = (xv[u].z * inv) * wv[u].z;
      yr[4 * i4 + 3] = (xv[u].w * inv) * wv[u].w;
    }
  }
  if (tid < tail) yr[4 * nq + tid] = (xr[4 * nq + tid] * inv) * w[4 * nq + tid];
}

// ---------------------------------------------------------------- attention

// dot_f32_scalar (kernels_cpu.cpp:30-43) of q (LDS) and one cached key row
__device__ __forceinline__ float dot4(const float* __restrict__ a, const float* __restrict__ b, int k) {
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  int i = 0;
  for (; i + 4 <= k; i += 4) {
    const float4 bv = *reinterpret_cast<const float4*>(b + i);
    s0 = s0 + a[i] * bv.x;
    s1 = s1 + a[i + 1] * bv.y;
    s2 = s2 + a[i + 2] * bv.z;
    s3 = s3 + a[i + 3] * bv.w;
  }
  for (; i < k; ++i) s0 = s0 + a[i] * b[i];
  return (s0 + s1) + (s2 + s3);
}

// Step 1 of cpu::attention: this step's keys (rotated when cos/sin are given) and values go to the
// cache [kv_head][pos][hd]. One workgroup per (token, kv head). pos_dev (if not null) holds pos0 in
// device memory, so that a captured decode step replays at any position.
__global__ __launch_bounds__(64) void kv_append_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                       float* __restrict__ kc, float* __restrict__ vc, int pos0,
                                                       const int* __restrict__ pos_dev, int n_kv, int hd, int max_ctx,
                                                       const float* __restrict__ rcos, const float* __restrict__ rsin) {
  if (pos_dev) pos0 = min(max(*pos_dev, 0), max_ctx - 1);  // the caller keeps it in range; stay in bounds anyway
  const int t = blockIdx.x / n_kv, h = blockIdx.x - t * n_kv, pos = pos0 + t, h2 = hd / 2;
  const float* ks = k + ((int64_t)t * n_kv + h) * hd;
  const float* vs = v + ((int64_t)t * n_kv + h) * hd;
  float* kd = kc + ((int64_t)h * max_ctx + pos) * hd;
  float* vd = vc + ((int64_t)h * max_ctx + pos) * hd;
  if (rcos) {
    const float* c = rcos + (int64_t)pos * h2;
    const float* s = rsin + (int64_t)pos * h2;
    for (int i = threadIdx.x; i < h2; i += 64) {
      kd[i] = ks[i] * c[i] - ks[i + h2] * s[i];
      kd[i + h2] = ks[i + h2] * c[i] + ks[i] * s[i];
    }
  } else {
    for (int i = threadIdx.x; i < hd; i += 64) kd[i] = ks[i];
  }
  for (int i = threadIdx.x; i < hd; i += 64) vd[i] = vs[i];
}

// Step 2 of cpu::attention: one 256-thread workgroup per (query token t, head h) over positions
// 0 .. pos0 + t, every float operation in cpu::attention's order:
//   q rotated into LDS; thread j computes sc[j] = dot_f32(q, k_j) * scale (its key row's loads all
//   in flight at once); mx = max sc; e_j = expf(sc[j] - mx); thread 0 sums e_0 + e_1 + ... in
//   order, inv = 1 / sum; p_j = e_j * inv; o_i = 0, o_i += p_j * v_j[i] in increasing j.
// Only the two sums are chains. The products p_j * v_j[i] are independent roundings: every
// thread forms them for its float4s of values (each value loaded once, straight from the cache)
// and writes them to LDS as rows of hd, so that lane i of wave 0 then only adds, reading row j's
// element i (64 consecutive floats: no bank conflict), 16 positions per batch with the next
// batch's reads issued before this batch's adds. Values move in chunks of whole positions (a
// multiple of 16), kAttnVF float4 per thread; the first chunk's loads are issued at the start,
// after q's and the key row's, and chunk c + 1 is loaded into registers while wave 0 adds chunk
// c. Every load is unconditional (indices clamped), so waiting for the first ones does not wait
// for the later ones. Score slots past the last position hold +0.0 and product rows past it are
// zero: adding them changes no sum (these sums start at +0.0 and are never -0.0).
// LDS (dynamic): q [hd], scores [n_cap rounded up to 64], one product chunk [cpos][hd].
// GS (global scores): for score rows longer than LDS holds, the row lives in gsc (one row of n_cap
// rounded up to 64 floats per workgroup) and LDS keeps q and the product chunk only; the in-order sum
// of the exponentials then passes them through the product region a chunk at a time. Same float
// operations in the same order.
constexpr int kAttnThreads = 256;
constexpr int kAttnVF = 20;                           // float4 of values per thread per chunk
constexpr int kAttnChunkF4 = kAttnThreads * kAttnVF;  // 80 KB: 320 positions of head size 64

__device__ __host__ __forceinline__ int attn_chunk_pos(int hd) { return (kAttnChunkF4 / (hd / 4)) & ~15; }

__device__ __forceinline__ float dot_row(const float* __restrict__ q, const float* __restrict__ k, int hd) {
  if (hd == 64) {  // the common head size: all 16 loads issued before the first product
    float4 kv[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) kv[u] = reinterpret_cast<const float4*>(k)[u];
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      s0 = s0 + q[4 * u] * kv[u].x;
      s1 = s1 + q[4 * u + 1] * kv[u].y;
      s2 = s2 + q[4 * u + 2] * kv[u].z;
      s3 = s3 + q[4 * u + 3] * kv[u].w;
    }
    return (s0 + s1) + (s2 + s3);
  }
  return dot4(q, k, hd);
}

// HD: the head size when it is known at compile time (64), else 0 (hd_arg). GS: scores in gsc.
template <int HD, bool GS>
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(const float* __restrict__ q, float* __restrict__ out,
                                                                 float* __restrict__ kc, float* __restrict__ vc, int pos0,
                                                                 const int* __restrict__ pos_dev, int n_heads, int n_kv,
                                                                 int hd_arg, int max_ctx, int n_cap,
                                                                 const float* __restrict__ rcos,
                                                                 const float* __restrict__ rsin,
                                                                 const float* __restrict__ knew,
                                                                 const float* __restrict__ vnew,
                                                                 float* __restrict__ gsc) {
  const int hd = HD ? HD : hd_arg;
  extern __shared__ float lds[];
  if (pos_dev) pos0 = min(max(*pos_dev, 0), max_ctx - 1);  // the caller keeps it in range; stay in bounds anyway
  const int hdp = (hd + 3) & ~3;
  const int row = (n_cap + 63) & ~63;  // score slots
  float* qb = lds;
  float* sc = GS ? gsc + (int64_t)blockIdx.x * row : lds + hdp;
  float* vt = GS ? lds + hdp : sc + row;
  float* kn = vt + attn_chunk_pos(hd) * hd;  // fused append: this step's rotated key
  __shared__ float red[kAttnThreads / 64];
  __shared__ float inv_s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t = blockIdx.x / n_heads, h = blockIdx.x - t * n_heads, pos = pos0 + t, h2 = hd / 2, n = pos + 1;
  const int qd = n_heads * hd, grp = n_heads / n_kv;
  // q first: the rotation needs it before anything else
  const float* qs = q + (int64_t)t * qd + h * hd;
  float qa = 0.f, qb2 = 0.f, cr = 0.f, sr = 0.f;
  const int iq = tid < hd ? tid : 0;
  if (rcos) {
    const int ih = tid < h2 ? tid : 0;
    qa = qs[ih];
    qb2 = qs[ih + h2];
    cr = rcos[(int64_t)pos * h2 + ih];
    sr = rsin[(int64_t)pos * h2 + ih];
  } else {
    qa = qs[iq];
  }
  const int kvh = h / grp;
  const float* kh = kc + (int64_t)kvh * max_ctx * hd;
  const v4f* vh4 = reinterpret_cast<const v4f*>(vc + (int64_t)kvh * max_ctx * hd);
  const int hd4 = hd / 4, cpos = attn_chunk_pos(hd), cf4 = cpos * hd4;
  const int total4 = n * hd4;  // the values to read, as float4 (hd % 4 == 0)
  // With the append fused (one decode token: knew / vnew given), the last position's key comes
  // from knew (rotated, through LDS) and its value from vnew, and the cache reads stop one row
  // earlier (that row is being written by another workgroup of the kv group).
  const bool fuse = knew != nullptr;
  const int nc = fuse ? max(n - 1, 1) : n;  // cache rows read
  float ka = 0.f, kb = 0.f, va = 0.f, vb = 0.f;
  if (fuse) {
    const float* ks = knew + kvh * hd;
    const float* vs = vnew + kvh * hd;
    const int ih = tid < h2 ? tid : 0;
    ka = ks[ih];
    kb = ks[ih + h2];
    va = vs[ih];
    vb = vs[ih + h2];  // for the cache write
  }
  // head size 64: this thread's first key row in flight from the start
  float4 kr[16];
  if (hd == 64) {  // fused: the last position's row is knew's (rotated below, before its score)
    const float* krow = fuse && tid == n - 1 ? knew + kvh * hd : kh + (int64_t)min(tid, nc - 1) * hd;
    const float4* k4 = reinterpret_cast<const float4*>(krow);
#pragma unroll
    for (int u = 0; u < 16; ++u) kr[u] = k4[u];
  }
  // chunk 0 of the values, also in flight from the start; with the append fused, the last
  // position's float4s are read from vnew (one load either way: the address is selected)
  const v4f* vnb = fuse ? reinterpret_cast<const v4f*>(vnew + kvh * hd) : vh4;
  auto vsrc = [&](int f) {
    const int fl = f - (n - 1) * hd4;
    return fuse && fl >= 0 ? vnb + fl : vh4 + f;
  };
  v4f vr[kAttnVF];
#pragma unroll
  for (int u = 0; u < kAttnVF; ++u) vr[u] = *vsrc(min(tid + u * kAttnThreads, total4 - 1));
  if (rcos) {
    if (tid < h2) {
      qb[tid] = qa * cr - qb2 * sr;
      qb[tid + h2] = qb2 * cr + qa * sr;
    }
  } else if (tid < hd) {
    qb[tid] = qa;
  }
  if (fuse && tid < h2) {
    // step 1 of cpu::attention for this token (kv_append_kernel's arithmetic): the rotated key into
    // LDS, key and value into the cache by the kv group's first workgroup
    const float k0 = rcos ? ka * cr - kb * sr : ka, k1 = rcos ? kb * cr + ka * sr : kb;
    kn[tid] = k0;
    kn[tid + h2] = k1;
    if (h % grp == 0) {
      float* kd = kc + ((int64_t)kvh * max_ctx + pos) * hd;
      float* vd = vc + ((int64_t)kvh * max_ctx + pos) * hd;
      kd[tid] = k0;
      kd[tid + h2] = k1;
      vd[tid] = va;
      vd[tid + h2] = vb;
    }
  }
  __syncthreads();
  const float scale = 1.0f / sqrtf((float)hd);
  float mx = -INFINITY;
  for (int j = tid; j < n; j += kAttnThreads) {
    float d;
    if (hd == 64 && fuse && rcos && j == n - 1 && j == tid) {
      // this step's key, preloaded unrotated: kv_append_kernel's rotation of pairs (i, i + 32)
      const float4* c4 = reinterpret_cast<const float4*>(rcos + (int64_t)pos * h2);
      const float4* s4 = reinterpret_cast<const float4*>(rsin + (int64_t)pos * h2);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float4 cc = c4[u], ss = s4[u], ka4 = kr[u], kb4 = kr[u + 8];
        kr[u] = make_float4(ka4.x * cc.x - kb4.x * ss.x, ka4.y * cc.y - kb4.y * ss.y, ka4.z * cc.z - kb4.z * ss.z,
                            ka4.w * cc.w - kb4.w * ss.w);
        kr[u + 8] = make_float4(kb4.x * cc.x + ka4.x * ss.x, kb4.y * cc.y + ka4.y * ss.y, kb4.z * cc.z + ka4.z * ss.z,
                                kb4.w * cc.w + ka4.w * ss.w);
      }
    }
    if (fuse && j == n - 1 && !(hd == 64 && j == tid)) {  // the step's key from LDS
      d = dot4(qb, kn, hd);
    } else if (hd == 64 && j == tid) {  // the preloaded row: dot_f32_scalar's order
      float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        s0 = s0 + qb[4 * u] * kr[u].x;
        s1 = s1 + qb[4 * u + 1] * kr[u].y;
        s2 = s2 + qb[4 * u + 2] * kr[u].z;
        s3 = s3 + qb[4 * u + 3] * kr[u].w;
      }
      d = (s0 + s1) + (s2 + s3);
    } else {
      d = dot_row(qb, kh + (int64_t)j * hd, hd);
    }
    const float sj = d * scale;
    sc[j] = sj;
    mx = fmaxf(mx, sj);
  }
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // e_j, and +0.0 in the slots up to the next multiple of 64
  const int n64 = (n + 63) & ~63;
  for (int j = tid; j < n64; j += kAttnThreads) sc[j] = j < n ? elm_expf(sc[j] - mx) : 0.f;
  __syncthreads();
  // e_0 + e_1 + ... in order by thread 0, 64 values read from LDS before their adds
  auto add_in_order = [](float sum, const float* e_lds, int count) {
    const float4* s4 = reinterpret_cast<const float4*>(e_lds);
    for (int j0 = 0; j0 < count; j0 += 64) {
      float4 e[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) e[u] = s4[(j0 >> 2) + u];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        sum = sum + e[u].x;
        sum = sum + e[u].y;
        sum = sum + e[u].z;
        sum = sum + e[u].w;
      }
    }
    return sum;
  };
  if (GS) {
    // the row passes through the product region (a multiple of 64 floats) a chunk at a time
    const int ch = attn_chunk_pos(hd) * hd;
    float sum = 0.f;
    for (int c0 = 0; c0 < n; c0 += ch) {
      const int m = min(ch, n64 - c0);
      for (int i = 4 * tid; i < m; i += 4 * kAttnThreads)
        *reinterpret_cast<float4*>(vt + i) = *reinterpret_cast<const float4*>(sc + c0 + i);
      __syncthreads();
      if (tid == 0) sum = add_in_order(sum, vt, min(ch, n - c0));
      __syncthreads();
    }
    if (tid == 0) inv_s = 1.0f / sum;
  } else if (tid == 0) {
    inv_s = 1.0f / add_in_order(0.f, sc, n);
  }
  __syncthreads();
  const float inv = inv_s;
  // The products p_j * v_j[i] of a chunk, p_j = e_j * inv, into LDS as rows of hd (this thread's
  // float4 of values: position j, dims 4 d .. 4 d + 3); zero rows past the last position.
  v4f* vt4 = reinterpret_cast<v4f*>(vt);
  auto products = [&](int f) {
    // only the rows the accumulation reads: this chunk's positions, zero-padded to a multiple of 16
    const int lim = min(cf4, ((min(cpos, n - f / hd4) + 15) & ~15) * hd4);
    float e[kAttnVF];  // every e_j first (slots past the last position read +0.0), then the products
#pragma unroll
    for (int u = 0; u < kAttnVF; ++u) e[u] = sc[min((f + tid + u * kAttnThreads) / hd4, n64 - 1)];
#pragma unroll
    for (int u = 0; u < kAttnVF; ++u) {
      const int rel = tid + u * kAttnThreads;
      if (rel < lim) {
        const float pj = e[u] * inv;
        const v4f pr = v4f{pj * vr[u].x, pj * vr[u].y, pj * vr[u].z, pj * vr[u].w};
        vt4[rel] = f + rel < total4 ? pr : v4f{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  products(0);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};  // wave 0: outputs lane, lane + 64, ... (hd <= 256)
  for (int f0 = 0; f0 < total4; f0 += cf4) {
    const int fn = f0 + cf4;
    if (fn < total4) {  // the next chunk into registers while this one is accumulated
#pragma unroll
      for (int u = 0; u < kAttnVF; ++u) vr[u] = *vsrc(min(fn + tid + u * kAttnThreads, total4 - 1));
    }
    __syncthreads();  // this chunk's products are in LDS
    if (wave == 0) {
      // positions j0 .. j0 + m - 1 in batches of 16 (chunks hold a multiple of 16 positions; the
      // rows past the last position are zero); the next batch's reads go out before this one's adds
      const int j0 = f0 / hd4, m = min(cpos, n - j0), nbat = (m + 15) >> 4;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = lane + 64 * r;
        if (i < hd) {
          float a = acc[r];
          auto load = [&](int bt, float (&vv)[16]) {
            const int jj = min(bt, nbat - 1) * 16;
#pragma unroll
            for (int u = 0; u < 16; ++u) vv[u] = vt[(jj + u) * hd + i];
          };
          auto fold = [&](const float (&vv)[16]) {
#pragma unroll
            for (int u = 0; u < 16; ++u) a = a + vv[u];
          };
          float va[16], vb[16];
          load(0, va);
          for (int bt = 0; bt < nbat; bt += 2) {
            load(bt + 1, vb);
            __builtin_amdgcn_sched_barrier(0);
            fold(va);
            if (bt + 1 < nbat) {
              load(bt + 2, va);
              __builtin_amdgcn_sched_barrier(0);
              fold(vb);
            }
          }
          acc[r] = a;
        }
      }
    }
    if (fn < total4) {
      __syncthreads();  // wave 0 is done with this chunk
      products(fn);
    }
  }
  float* o = out + (int64_t)t * qd + h * hd;
  if (wave == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (lane + 64 * r < hd) o[lane + 64 * r] = acc[r];
  }
}

// Decode (one token, head size 64, the append fused): attention_kernel's float operations in the
// same order (cpu::attention), with the cached rows moved into LDS by DMA, whole rows per
// instruction, instead of each thread loading its own key row and a share of the values (loads
// that touch a different line in every lane). One 256-thread workgroup per head:
//  - key rows [0, C) of the kv head go to LDS first, before the position has arrived; the rows
//    past the step's are stale cache contents and are never used (every row read lies below
//    max_ctx). The 16-byte slot s of row r holds the row's chunk s ^ (r & 15), so that lanes
//    reading chunk u of consecutive rows hit different bank groups;
//  - the value rows [0, C) follow once q is rotated and land while the scores, their max, the
//    exponentials and their sum run;
//  - thread j scores row j (position n - 1: the step's own key, rotated, from LDS); wave 0 sums
//    the exponentials in order (ordered_sum256); p_j = e_j * inv is formed once per position;
//    lane i of wave 0 then adds p_j * v_j[i] over the value rows in LDS in increasing j, the
//    step's own value (from registers) last.
// Against attention_kernel at 200 positions this takes ~7 us instead of ~9.3 us inside a graph.
// Caches longer than C rows pass through the same buffers a chunk at a time: keys through the key
// buffer, values alternating between both, the next chunk in flight while wave 0 adds the current.
// LDS (dynamic): keys [C][64], values [C][64], scores [n_cap rounded up to 256], q [64], the
// step's rotated key [64].
constexpr int kDecRows = 256;  // C: rows per LDS buffer, one per thread

// dot_f32_scalar's order (four strided accumulators, then (s0 + s1) + (s2 + s3)) of q and a row
// in LDS whose chunk u sits in slot u ^ swz
__device__ __forceinline__ float dot64_lds(const float* __restrict__ q, const float* __restrict__ row, int swz) {
  float4 kv[16];
#pragma unroll
  for (int u = 0; u < 16; ++u) kv[u] = *reinterpret_cast<const float4*>(row + ((u ^ swz) << 2));
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    s0 = s0 + q[4 * u] * kv[u].x;
    s1 = s1 + q[4 * u + 1] * kv[u].y;
    s2 = s2 + q[4 * u + 2] * kv[u].z;
    s3 = s3 + q[4 * u + 3] * kv[u].w;
  }
  return (s0 + s1) + (s2 + s3);
}

// acc + p_0 v_0 + p_1 v_1 + ... + p_{n-1} v_{n-1} in order (n <= 16 NB): each product rounded, then
// added (cpu::attention's o_i += p_j * v_j[i] without contraction), p_j = pj[j] and v_j = vcol[64 j];
// the reads stay below 16 NB values of each. Straight-line code over batches of 16, as
// ordered_sum256: batch b + 2 is read and batch b + 1's products are formed while batch b's
// products are added, so the dependent adds alternate with independent multiplies (the empty asm
// keeps each product in its step instead of sunk to the step that adds it). The last, partial
// batch is added from the same registers, the products past n replaced by +0.0: acc starts at +0.0
// and a sum of floats that starts at +0.0 is never -0.0 (x + y = -0.0 needs x = y = -0.0), so each
// of those adds leaves acc unchanged (one loop step per position with its own LDS round trip cost
// up to 0.5 us for the last 15 positions).
template <int NB>
__device__ __forceinline__ float ordered_dot_col(const float* __restrict__ pj, const float* __restrict__ vcol, int n,
                                                 float acc) {
  const int nbt = n >> 4, rem = n & 15;
  float pv[3][16], xv[3][16], pr[2][16], tl[16];
#define ELM_DOT_LOAD(bt)                                                                           \
  _Pragma("unroll") for (int u = 0; u < 16; ++u) {                                                 \
    pv[(bt) % 3][u] = pj[16 * (bt) + u];                                                           \
    xv[(bt) % 3][u] = vcol[64 * (16 * (bt) + u)];                                                  \
  }                                                                                                \
  asm volatile("" ::: "memory");
#define ELM_DOT_STEP(bt)                                                                           \
  if (nbt <= (bt)) {                                                                               \
    _Pragma("unroll") for (int u = 0; u < 16; ++u) tl[u] = pr[(bt) % 2][u];                        \
    goto tail;                                                                                     \
  }                                                                                                \
  if ((bt) + 2 < NB) { ELM_DOT_LOAD((bt) + 2) }                                                    \
  _Pragma("unroll") for (int u = 0; u < 16; ++u) {                                                 \
    if ((bt) + 1 < NB) {                                                                           \
      pr[((bt) + 1) % 2][u] = pv[((bt) + 1) % 3][u] * xv[((bt) + 1) % 3][u];                       \
      asm volatile("" : "+v"(pr[((bt) + 1) % 2][u]));                                              \
    }                                                                                              \
    acc = acc + pr[(bt) % 2][u];                                                                   \
  }
  ELM_DOT_LOAD(0)
  if (NB > 1) { ELM_DOT_LOAD(1) }
#pragma unroll
  for (int u = 0; u < 16; ++u) pr[0][u] = pv[0][u] * xv[0][u];
  ELM_DOT_STEP(0)
  if (NB > 1) { ELM_DOT_STEP(1) }
  if (NB > 2) { ELM_DOT_STEP(2) }
  if (NB > 3) { ELM_DOT_STEP(3) }
  if (NB > 4) { ELM_DOT_STEP(4) }
  if (NB > 5) { ELM_DOT_STEP(5) }
  if (NB > 6) { ELM_DOT_STEP(6) }
  if (NB > 7) { ELM_DOT_STEP(7) }
  if (NB > 8) { ELM_DOT_STEP(8) }
  if (NB > 9) { ELM_DOT_STEP(9) }
  if (NB > 10) { ELM_DOT_STEP(10) }
  if (NB > 11) { ELM_DOT_STEP(11) }
  if (NB > 12) { ELM_DOT_STEP(12) }
  if (NB > 13) { ELM_DOT_STEP(13) }
  if (NB > 14) { ELM_DOT_STEP(14) }
  if (NB > 15) { ELM_DOT_STEP(15) }
#undef ELM_DOT_STEP
#undef ELM_DOT_LOAD
  return acc;
tail:
  if (rem > 0) {
#pragma unroll
    for (int u = 0; u < 16; ++u) acc = acc + (u < rem ? tl[u] : 0.f);
  }
  return acc;
}

__global__ __launch_bounds__(256) void attention_decode64_kernel(
    const float* __restrict__ q, float* __restrict__ out, float* __restrict__ kc, float* __restrict__ vc, int pos0,
    const int* __restrict__ pos_dev, int grp, int n_kv, int max_ctx, int n_cap, const float* __restrict__ rcos,
    const float* __restrict__ rsin, const float* __restrict__ knew, const float* __restrict__ vnew) {
  constexpr int HD = 64, H2 = 32, C = kDecRows, ROWB = HD * 4;
  // Every argument into scalar registers before anything else: their loads go out as one batch, so the
  // first memory requests wait for one round trip to the argument segment (loaded near their first
  // uses instead, they took three, one behind the other).
  asm volatile("" ::"s"(q), "s"(out), "s"(kc), "s"(vc), "s"(pos0), "s"(pos_dev), "s"(grp), "s"(n_kv),
               "s"(max_ctx), "s"(n_cap), "s"(rcos), "s"(rsin), "s"(knew), "s"(vnew));
  extern __shared__ __align__(16) float lds[];
  float* const kb = lds;
  float* const vb = kb + C * HD;
  float* const sc = vb + C * HD;
  float* const qb = sc + ((n_cap + 255) & ~255);
  float* const kn = qb + HD;
  __shared__ float red[4];
  __shared__ float inv_s;
  // the wave index as a scalar: loops over it stay scalar loops instead of divergent ones
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // workgroup (kv head, head of its group): the grid is n_kv x grp (grp = n_heads / n_kv, passed in),
  // so the head needs no division
  const int kvh = blockIdx.x, h = kvh * grp + blockIdx.y;
  const float* const kh = kc + (int64_t)kvh * max_ctx * HD;
  const float* const vh = vc + (int64_t)kvh * max_ctx * HD;
  const unsigned kb_lds = (unsigned)(size_t)(LdsBytes)(unsigned char*)kb;
  const unsigned vb_lds = (unsigned)(size_t)(LdsBytes)(unsigned char*)vb;
  // the position's load goes out first and is waited for only after the key rows' requests
  // (without pos_dev it reads q's first word, in bounds, and ignores it); then this step's q, key
  // and value pairs (i, i + 32) and lane's element of the value
  const int pos_raw = *(pos_dev ? pos_dev : reinterpret_cast<const int*>(q));
  const int ih = tid & (H2 - 1);
  const float* const qs = q + h * HD;
  const float* const ks = knew + kvh * HD;
  const float* const vs = vnew + kvh * HD;
  const float qa = qs[ih], qz = qs[ih + H2], ka = ks[ih], kz = ks[ih + H2], va = vs[ih], vz = vs[ih + H2];
  const float vlast = vs[lane];
  // key rows [0, CS) before the position is known: wave w moves 1 KB pieces w, w + 4, ... (4 rows
  // each, lane -> row lane / 16, slot lane % 16); rows past RS - 1 repeat it
  constexpr int CS = C / 2;
  const int RS = min(CS, max_ctx);
#pragma unroll
  for (int i = 0; i < CS / 16; ++i) {
    const int pc = wave + 4 * i, r = 4 * pc + (lane >> 4), s = lane & 15;
    dma16s(kh, (uint32_t)(min(r, RS - 1) * ROWB + ((s ^ (r & 15)) << 4)), kb_lds + pc * 1024);
  }
  __builtin_amdgcn_sched_barrier(0);
  // the caller keeps the position in range; stay in bounds anyway
  const int pos = pos_dev ? min(max(pos_raw, 0), max_ctx - 1) : pos0;
  float cr = 0.f, sr = 0.f;
  if (rcos) {
    cr = rcos[(int64_t)pos * H2 + ih];
    sr = rsin[(int64_t)pos * H2 + ih];
  }
  // the first chunk's other cache rows, [CS, min(C, pos)), now that the position is known (the
  // last piece repeats row min(C, pos) - 1)
  const int n = pos + 1, nc = n - 1, rk = min(C, nc);
  for (int pc = CS / 4 + wave; 4 * pc < rk; pc += 4) {
    const int r = 4 * pc + (lane >> 4), s = lane & 15;
    dma16s(kh, (uint32_t)(min(r, rk - 1) * ROWB + ((s ^ (r & 15)) << 4)), kb_lds + pc * 1024);
  }
  wait_vm<0>();  // the keys, q, k, v and the rotation's cos / sin
  if (tid < H2) {
    // cpu::attention step 1 (kv_append_kernel's arithmetic) and q's rotation
    const float q0 = rcos ? qa * cr - qz * sr : qa, q1 = rcos ? qz * cr + qa * sr : qz;
    const float k0 = rcos ? ka * cr - kz * sr : ka, k1 = rcos ? kz * cr + ka * sr : kz;
    qb[tid] = q0;
    qb[tid + H2] = q1;
    kn[tid] = k0;
    kn[tid + H2] = k1;
    if (blockIdx.y == 0) {  // the kv group's first workgroup appends to the cache
      float* const kd = kc + ((int64_t)kvh * max_ctx + pos) * HD;
      float* const vd = vc + ((int64_t)kvh * max_ctx + pos) * HD;
      kd[tid] = k0;
      kd[tid + H2] = k1;
      vd[tid] = va;
      vd[tid + H2] = vz;
    }
  }
  lds_barrier();  // keys (every wave waited for its own), q and the step's key in LDS

  // scores: thread j takes row j of each chunk of C positions; the cache rows are 0 .. n - 2
  const float scale = 1.0f / sqrtf((float)HD);
  float mx = -INFINITY;
  for (int c0 = 0; c0 < n; c0 += C) {
    if (c0 > 0) {  // the next key chunk, once every thread has scored the previous one
      __syncthreads();
      const int rows = min(C, nc - c0);
      for (int pc = wave; 4 * pc < rows; pc += 4) {
        const int r = 4 * pc + (lane >> 4), s = lane & 15;
        dma16s(kh, (uint32_t)((c0 + min(r, rows - 1)) * ROWB + ((s ^ (r & 15)) << 4)), kb_lds + pc * 1024);
      }
      wait_vm<0>();
      lds_barrier();
    }
    const int j = c0 + tid;
    if (j < n) {
      const float d = j == nc ? dot64_lds(qb, kn, 0) : dot64_lds(qb, kb + tid * HD, tid & 15);
      const float sj = d * scale;
      sc[j] = sj;
      mx = fmaxf(mx, sj);
    }
  }
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // e_j, and +0.0 in the slots up to the next multiple of 16
  const int n16 = (n + 15) & ~15;
  for (int j = tid; j < n16; j += 256) sc[j] = j < n ? elm_expf(sc[j] - mx) : 0.f;
  __syncthreads();
  if (wave == 0) {  // e_0 + e_1 + ... in order (every lane runs the chain; lane 0 keeps the result)
    float sum = 0.f;
    for (int g0 = 0; g0 < n16; g0 += 256) sum = ordered_sum256(sc + g0, min(16, (n16 - g0) >> 4), sum);
    if (lane == 0) inv_s = 1.0f / sum;
  } else {
    // meanwhile waves 1-3 request the first chunk's value rows [0, min(C, n - 1)) into the value
    // buffer (unswizzled: lane i of wave 0 reads element i of a row; the last piece repeats the
    // last row): the key buffer may still hold the last key chunk, the value buffer is unused
    for (int pc = wave - 1; 4 * pc < rk; pc += 3) {
      const int r = 4 * pc + (lane >> 4);
      dma16s(vh, (uint32_t)(min(r, rk - 1) * ROWB + ((lane & 15) << 4)), vb_lds + pc * 1024);
    }
  }
  __syncthreads();
  const float inv = inv_s;
  for (int j = tid; j < n16; j += 256) sc[j] = sc[j] * inv;  // p_j
  wait_vm<0>();  // this wave's value rows
  __syncthreads();

  // o_i = 0, o_i += p_j * v_j[i] in increasing j: lane i of wave 0, value chunks of C rows
  // alternating between the two buffers, the next chunk in flight while wave 0 adds the current
  float acc = 0.f;
  for (int c0 = 0, ci = 0; c0 < nc; c0 += C, ++ci) {
    const float* const cur = (ci & 1) ? kb : vb;
    const int nx = c0 + C;
    if (nx < nc) {  // the next chunk into the other buffer (the keys' or the chunk before this one's)
      const int rows = min(C, nc - nx);
      const unsigned dst = (ci & 1) ? vb_lds : kb_lds;
      for (int pc = wave; 4 * pc < rows; pc += 4) {
        const int r = 4 * pc + (lane >> 4);
        dma16s(vh, (uint32_t)((nx + min(r, rows - 1)) * ROWB + ((lane & 15) << 4)), dst + pc * 1024);
      }
    }
    if (wave == 0) {  // 16 positions per batch (C / 16 at most), the last batch partial
      const int m = min(C, nc - c0);
      acc = ordered_dot_col<kDecRows / 16>(sc + c0, cur + lane, m, acc);
    }
    if (nx < nc) {
      wait_vm<0>();
      __syncthreads();
    }
  }
  if (wave == 0) out[h * HD + lane] = acc + sc[nc] * vlast;  // position n - 1: the step's own value
}

// Prefill (T > 1, head size 64): one workgroup per (head, kAttnQ consecutive query tokens), wave w
// for query t0 + w. Keys and values are read once for the group's queries instead of once per
// query, and the per-query chains (the sum of the exponentials, lane 0; the 64 output sums, one
// per lane) run in the four waves at once. Same float operations in the same order as
// attention_kernel (cpu::attention): scores by dot_f32_scalar's order, max, expf(s - max), the sum
// in increasing position, p_j = e_j * inv, o_i += p_j * v_j[i] in increasing position.
// LDS (dynamic): q [kAttnQ][64], scores [kAttnQ][n_cap rounded up to 64], values [kAttnPVPos][64].
constexpr int kAttnQ = 4;
constexpr int kAttnPVPos = 96;  // value rows per chunk (24 KB)

__global__ __launch_bounds__(256) void attention_prefill_kernel(const float* __restrict__ q, float* __restrict__ out,
                                                                const float* __restrict__ kc,
                                                                const float* __restrict__ vc, int pos0, int T,
                                                                int n_heads, int n_kv, int max_ctx, int n_cap,
                                                                const float* __restrict__ rcos,
                                                                const float* __restrict__ rsin,
                                                                int8_t* __restrict__ xq, float* __restrict__ xd,
                                                                int Tpad) {
  constexpr int hd = 64, h2 = 32, hd4 = 16;
  extern __shared__ float lds[];
  const int scs = (n_cap + 63) & ~63;  // score row stride
  float* qb = lds;                     // [kAttnQ][64]
  float* sc = qb + kAttnQ * hd;        // [kAttnQ][scs]
  float* vt = sc + kAttnQ * scs;       // [kAttnPVPos][64]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int ngr = (T + kAttnQ - 1) / kAttnQ;
  const int h = blockIdx.x / ngr, t0 = (blockIdx.x - h * ngr) * kAttnQ;
  const int nq = min(kAttnQ, T - t0);               // queries in this group
  const int tw = t0 + min(w, nq - 1), posw = pos0 + tw, nw = posw + 1;  // this wave's query
  const int nmax = pos0 + t0 + nq;                  // positions of the group's last query
  const int qd = n_heads * hd, grp = n_heads / n_kv, kvh = h / grp;
  const float* kh = kc + (int64_t)kvh * max_ctx * hd;
  const float4* vh4 = reinterpret_cast<const float4*>(vc + (int64_t)kvh * max_ctx * hd);
  // 1. q of the wave's query, rotated, into LDS
  {
    const float* qs = q + (int64_t)tw * qd + h * hd;
    if (rcos) {
      if (lane < h2) {
        const float a = qs[lane], b = qs[lane + h2];
        const float c = rcos[(int64_t)posw * h2 + lane], sn = rsin[(int64_t)posw * h2 + lane];
        qb[w * hd + lane] = a * c - b * sn;
        qb[w * hd + lane + h2] = b * c + a * sn;
      }
    } else {
      qb[w * hd + lane] = qs[lane];
    }
  }
  __syncthreads();
  // 2. scores: thread j takes positions j, j + 256, ...: one key row, the group's dot products
  const float scale = 1.0f / sqrtf((float)hd);
  for (int j = tid; j < nmax; j += 256) {
    float4 kr[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) kr[u] = reinterpret_cast<const float4*>(kh + (int64_t)j * hd)[u];
#pragma unroll
    for (int qi = 0; qi < kAttnQ; ++qi) {
      if (qi < nq && j <= pos0 + t0 + qi) {
        const float* qq = qb + qi * hd;
        float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          s0 = s0 + qq[4 * u] * kr[u].x;
          s1 = s1 + qq[4 * u + 1] * kr[u].y;
          s2 = s2 + qq[4 * u + 2] * kr[u].z;
          s3 = s3 + qq[4 * u + 3] * kr[u].w;
        }
        sc[qi * scs + j] = ((s0 + s1) + (s2 + s3)) * scale;
      }
    }
  }
  __syncthreads();
  // 3. per wave (query): max, exponentials (+0.0 past the last position, to a multiple of 64),
  // the in-order sum by lane 0, p_j = e_j * inv
  float* sw = sc + w * scs;
  float mx = -INFINITY;
  for (int j = lane; j < nw; j += 64) mx = fmaxf(mx, sw[j]);
  mx = wave_max(mx);
  const int n64 = (nw + 63) & ~63;
  for (int j = lane; j < n64; j += 64) sw[j] = j < nw ? elm_expf(sw[j] - mx) : 0.f;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  float sum = 0.f;
  if (lane == 0) {
    const float4* s4 = reinterpret_cast<const float4*>(sw);
    for (int j0 = 0; j0 < nw; j0 += 64) {
      float4 e[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) e[u] = s4[(j0 >> 2) + u];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        sum = sum + e[u].x;
        sum = sum + e[u].y;
        sum = sum + e[u].z;
        sum = sum + e[u].w;
      }
    }
  }
  const float inv = 1.0f / __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sum)));
  __builtin_amdgcn_wave_barrier();
  for (int j = lane; j < nw; j += 64) sw[j] = sw[j] * inv;
  // 4. values by chunks of whole positions into LDS (rows of 64; zero rows past the group's last
  // position), then each wave adds p_j * v_j[lane] for its own positions in increasing j
  float acc = 0.f;
  float4* vt4 = reinterpret_cast<float4*>(vt);
  for (int j0 = 0; j0 < nmax; j0 += kAttnPVPos) {
    __syncthreads();  // every p_j written (first chunk); the previous chunk consumed
    const int rows = min(kAttnPVPos, nmax - j0);
    for (int f = tid; f < kAttnPVPos * hd4; f += 256)
      vt4[f] = f < rows * hd4 ? vh4[(int64_t)j0 * hd4 + f] : make_float4(0.f, 0.f, 0.f, 0.f);
    __syncthreads();
    const int m = min(rows, nw - j0);  // this query's positions in the chunk
    auto batch = [&](int jj, int lim) {  // positions jj .. jj + 15, those below lim added
      float4 pv[4];
      float vv[16];
#pragma unroll
      for (int u = 0; u < 4; ++u) pv[u] = reinterpret_cast<const float4*>(sw + j0 + jj)[u];
#pragma unroll
      for (int u = 0; u < 16; ++u) vv[u] = vt[(jj + u) * hd + lane];
      const float pf[16] = {pv[0].x, pv[0].y, pv[0].z, pv[0].w, pv[1].x, pv[1].y, pv[1].z, pv[1].w,
                            pv[2].x, pv[2].y, pv[2].z, pv[2].w, pv[3].x, pv[3].y, pv[3].z, pv[3].w};
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (u < lim) acc = acc + pf[u] * vv[u];
    };
    int jj = 0;
    for (; jj + 16 <= m; jj += 16) batch(jj, 16);
    if (jj < m) batch(jj, m - jj);  // the last, partial batch
  }
  if (w < nq) {
    out[(int64_t)tw * qd + h * hd + lane] = acc;
    if (xq) {
      // the next GEMM's activation fragments: lanes 0-31 hold block 2h of token tw, lanes 32-63
      // block 2h + 1; scale = amax / 127 and edgelm's rounding, as act_quant_frag_kernel
      float a = fmaxf(0.f, fabsf(acc));
#pragma unroll
      for (int m = 1; m < 32; m <<= 1) a = fmaxf(a, __shfl_xor(a, m, 64));
      const float scl = a / 127.0f;
      int qv;
      elm_q8_group<1>(&acc, scl == 0.f ? 1.f : scl, &qv);
      const int b = 2 * h + (lane >> 5), e = lane & 31;
      xq[elm_frag_offset(tw, b, e >> 4, 2 * n_heads) + (e & 15)] = (int8_t)qv;
      if (e == 0) xd[(int64_t)b * Tpad + tw] = scl;
    }
  }
}

// Prefill (T > 1, head size 64) with the cached rows moved into LDS by DMA, as the decode kernel
// does: one 256-thread workgroup per (head, kAttnQ consecutive query tokens), wave w for query
// t0 + w; the same float operations in the same order as attention_prefill_kernel. Keys and
// values of positions [0, nmax) (nmax: the group's last query's positions) go to LDS kPfRows rows
// at a time: thread j scores row j against the group's queries; then each wave takes its own
// query's max, exponentials, in-order sum (ordered_sum256) and p_j = e_j * inv, and adds
// p_j * v_j[lane] over the value rows in increasing j. Longer prompts pass through the buffers a
// chunk at a time (keys through the key buffer; values alternating, the next chunk in flight).
// Step 1 of cpu::attention (the append) is part of the kernel: rows from pos0 on come from the
// step's own keys and values (knew, vnew: [T][n_kv][64]) instead of the cache, the keys rotated in
// LDS once they have landed (kv_append_kernel's arithmetic), and the workgroups of each kv group's
// first head write their query tokens' rotated keys and values to the cache (nothing in this
// launch reads them there).
// LDS (dynamic): keys [kPfRows][64] (chunk u of row r in slot u ^ (r & 15)), values [kPfRows][64],
// scores [kAttnQ][n_cap rounded up to 256], q [kAttnQ][64].
constexpr int kPfRows = 128;

__global__ __launch_bounds__(256) void attention_prefill64_kernel(
    const float* __restrict__ q, float* __restrict__ out, float* __restrict__ kc, float* __restrict__ vc, int pos0,
    int T, int grp, int n_kv, int max_ctx, int n_cap, const float* __restrict__ rcos, const float* __restrict__ rsin,
    int8_t* __restrict__ xq, float* __restrict__ xd, int Tpad, const float* __restrict__ knew,
    const float* __restrict__ vnew) {
  constexpr int HD = 64, H2 = 32, R = kPfRows, ROWB = HD * 4;
  // every argument into scalar registers first, in one batch of loads (as the decode kernel)
  asm volatile("" ::"s"(q), "s"(out), "s"(kc), "s"(vc), "s"(pos0), "s"(T), "s"(grp), "s"(n_kv), "s"(max_ctx),
               "s"(n_cap), "s"(rcos), "s"(rsin), "s"(xq), "s"(xd), "s"(Tpad), "s"(knew), "s"(vnew));
  extern __shared__ __align__(16) float lds[];
  const int scs = (n_cap + 255) & ~255;  // score row stride
  float* const kb = lds;                 // [R][64]
  float* const vb = kb + R * HD;         // [R][64]
  float* const sc = vb + R * HD;         // [kAttnQ][scs]
  float* const qb = sc + kAttnQ * scs;   // [kAttnQ][64]
  // the wave index as a scalar: loops over it stay scalar loops instead of divergent ones
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  // workgroup (query group, head of its kv group, kv head): the grid is ngr x grp x n_kv (grp =
  // n_heads / n_kv, passed in), so the head and kv head need no integer division
  const int kvh = blockIdx.z, h = kvh * grp + blockIdx.y, t0 = blockIdx.x * kAttnQ, n_heads = grp * n_kv;
  const int nq = min(kAttnQ, T - t0);                                   // queries in this group
  const int tw = t0 + min(w, nq - 1), posw = pos0 + tw, nw = posw + 1;  // this wave's query
  const int nmax = pos0 + t0 + nq;                                      // the group's positions
  const int qd = n_heads * HD;
  float* const kh = kc + (int64_t)kvh * max_ctx * HD;
  float* const vh = vc + (int64_t)kvh * max_ctx * HD;
  const bool fresh = knew != nullptr;  // rows from pos0 on: the step's keys and values, not the cache
  // rows [c0, c0 + rows) of a cache (or, from pos0 on, of the step's rows of kv head kvh) into a
  // buffer: wave w moves 1 KB pieces w, w + 4, ... (4 rows each, lane -> row lane / 16, slot
  // lane % 16); the last piece repeats the last row
  // (each lane's source is picked without a branch, so that the copies issue back to back)
  auto dma_rows = [&](const float* cache, const float* step, int c0, int rows, float* dst, bool swz) {
    if (!fresh || c0 >= pos0 || c0 + rows <= pos0) {
      // one source for the whole range (uniform): a scalar base and 32-bit lane offsets, a few
      // instructions per copy (the per-lane 64-bit source select costs ~90 ns per copy)
      const bool st = fresh && c0 >= pos0;
      const float* const base = st ? step + (int64_t)kvh * HD : cache;
      const int rstride = st ? n_kv * ROWB : ROWB, r00 = st ? c0 - pos0 : c0;
      const unsigned dbase = (unsigned)(size_t)(LdsBytes)(unsigned char*)dst;
      for (int pc = w; 4 * pc < rows; pc += 4) {
        const int r = 4 * pc + (lane >> 4), s = lane & 15;
        const int ch = swz ? s ^ (r & 15) : s;
        dma16s(base, (uint32_t)((r00 + min(r, rows - 1)) * rstride + (ch << 4)), dbase + pc * 1024);
      }
      return;
    }
    const int64_t sstride = (int64_t)n_kv * HD;
    const float* const sbase = (fresh ? step : cache) + (fresh ? (int64_t)kvh * HD - (int64_t)pos0 * sstride : 0);
    for (int pc = w; 4 * pc < rows; pc += 4) {
      const int r = 4 * pc + (lane >> 4), s = lane & 15, p = c0 + min(r, rows - 1);
      const int ch = (swz ? s ^ (r & 15) : s) * 4;
      const bool st = fresh && p >= pos0;
      const int64_t off = (int64_t)p * (st ? sstride : (int64_t)HD) + ch;
      const uint64_t src = st ? (uint64_t)(size_t)sbase : (uint64_t)(size_t)cache;
      dma16(reinterpret_cast<const float*>(src) + off, reinterpret_cast<unsigned char*>(dst) + pc * 1024);
    }
  };
  // the step's key rows of [c0, c0 + rows) rotated in place, pairs (i, i + 32): thread task
  // (row r, chunk pair u, u + 8), tasks tid, tid + 256, ...; cos / sin of the first chunk's tasks
  // are loaded at the start (cpre)
  constexpr int kRotTasks = R * 8 / 256;
  float4 cpre[kRotTasks][2];
  // Every task's pair is read before the first is written (the tasks' slots are disjoint), so the
  // reads wait for LDS once instead of once per task.
  auto rotate_rows = [&](int c0, int rows, bool pre) {
    float4 a[kRotTasks], b[kRotTasks];
#pragma unroll
    for (int m = 0; m < kRotTasks; ++m) {
      const int task = tid + 256 * m, r = task >> 3, u = task & 7;
      const float* const row = kb + min(r, rows - 1) * HD;
      a[m] = *reinterpret_cast<const float4*>(row + ((u ^ (r & 15)) << 2));
      b[m] = *reinterpret_cast<const float4*>(row + (((u + 8) ^ (r & 15)) << 2));
    }
#pragma unroll
    for (int m = 0; m < kRotTasks; ++m) {
      const int task = tid + 256 * m, r = task >> 3, u = task & 7, p = c0 + r;
      if (r < rows && p >= pos0) {
        float* const row = kb + r * HD;
        float4* const lo = reinterpret_cast<float4*>(row + ((u ^ (r & 15)) << 2));
        float4* const hi = reinterpret_cast<float4*>(row + (((u + 8) ^ (r & 15)) << 2));
        const float4 c = pre ? cpre[m][0] : *reinterpret_cast<const float4*>(rcos + (int64_t)p * H2 + 4 * u);
        const float4 sn = pre ? cpre[m][1] : *reinterpret_cast<const float4*>(rsin + (int64_t)p * H2 + 4 * u);
        const float4 x = a[m], y = b[m];
        *lo = make_float4(x.x * c.x - y.x * sn.x, x.y * c.y - y.y * sn.y, x.z * c.z - y.z * sn.z, x.w * c.w - y.w * sn.w);
        *hi = make_float4(y.x * c.x + x.x * sn.x, y.y * c.y + x.y * sn.y, y.z * c.z + x.z * sn.z, y.w * c.w + x.w * sn.w);
      }
    }
  };
  dma_rows(kh, knew, 0, min(R, nmax), kb, true);
  if (fresh && rcos) {
#pragma unroll
    for (int m = 0; m < kRotTasks; ++m) {
      const int task = tid + 256 * m, p = min(task >> 3, nmax - 1), u = task & 7;
      cpre[m][0] = *reinterpret_cast<const float4*>(rcos + (int64_t)p * H2 + 4 * u);
      cpre[m][1] = *reinterpret_cast<const float4*>(rsin + (int64_t)p * H2 + 4 * u);
    }
  }
  // the append: token t0 + w's key element `lane`, rotated, and its value (kv group's first head)
  const bool writer = fresh && blockIdx.y == 0 && w < nq;
  float ak = 0.f, ap = 0.f, ac = 1.f, as = 0.f, av = 0.f;
  if (writer) {
    const float* const ks = knew + ((int64_t)(t0 + w) * n_kv + kvh) * HD;
    ak = ks[lane];
    ap = ks[lane ^ H2];
    av = vnew[((int64_t)(t0 + w) * n_kv + kvh) * HD + lane];
    if (rcos) {
      ac = rcos[(int64_t)(pos0 + t0 + w) * H2 + (lane & (H2 - 1))];
      as = rsin[(int64_t)(pos0 + t0 + w) * H2 + (lane & (H2 - 1))];
    }
  }
  // q of the wave's query, rotated, into LDS
  {
    const float* const qs = q + (int64_t)tw * qd + h * HD;
    const int ih = lane & (H2 - 1);
    const float a = qs[ih], b = qs[ih + H2];
    float c = 0.f, sn = 0.f;
    if (rcos) {
      c = rcos[(int64_t)posw * H2 + ih];
      sn = rsin[(int64_t)posw * H2 + ih];
    }
    wait_vm<0>();  // the keys, q, cos / sin
    if (lane < H2) {
      qb[w * HD + lane] = rcos ? a * c - b * sn : a;
      qb[w * HD + lane + H2] = rcos ? b * c + a * sn : b;
    }
  }
  dma_rows(vh, vnew, 0, min(R, nmax), vb, false);
  lds_barrier();  // keys (every wave waited for its own) and the queries in LDS
  if (fresh && rcos) {
    rotate_rows(0, min(R, nmax), true);
    lds_barrier();
  }
  if (writer) {  // kv_append_kernel's arithmetic
    const int p = pos0 + t0 + w;
    const float kr = !rcos ? ak : lane < H2 ? ak * ac - ap * as : ak * ac + ap * as;
    kh[(int64_t)p * HD + lane] = kr;
    vh[(int64_t)p * HD + lane] = av;
  }

  // scores: thread (j, g) takes row j of each chunk of R positions against queries 2 g and 2 g + 1
  // of the group (those that see it)
  static_assert(R == 128 && kAttnQ == 4, "two threads per key row, two queries each");
  const float scale = 1.0f / sqrtf((float)HD);
  const int srow = tid & (R - 1), sq0 = 2 * (tid >> 7);
  // the wave's two queries in registers, read once (every lane reads the same values)
  float4 qv[2][16];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int u = 0; u < 16; ++u) qv[i][u] = *reinterpret_cast<const float4*>(qb + (sq0 + i) * HD + 4 * u);
  for (int c0 = 0; c0 < nmax; c0 += R) {
    if (c0 > 0) {  // the next key chunk, once every thread has scored the previous one
      __syncthreads();
      dma_rows(kh, knew, c0, min(R, nmax - c0), kb, true);
      wait_vm<0>();
      lds_barrier();
      if (fresh && rcos && c0 + R > pos0) {
        rotate_rows(c0, min(R, nmax - c0), false);
        lds_barrier();
      }
    }
    const int j = c0 + srow;
    if (j < nmax && j <= pos0 + t0 + min(sq0 + 1, nq - 1)) {
      const float* const row = kb + srow * HD;
      const int sw = srow & 15;
      float4 kv[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) kv[u] = *reinterpret_cast<const float4*>(row + ((u ^ sw) << 2));
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int qi = sq0 + i;
        if (qi < nq && j <= pos0 + t0 + qi) {
          float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
          for (int u = 0; u < 16; ++u) {
            s0 = s0 + qv[i][u].x * kv[u].x;
            s1 = s1 + qv[i][u].y * kv[u].y;
            s2 = s2 + qv[i][u].z * kv[u].z;
            s3 = s3 + qv[i][u].w * kv[u].w;
          }
          sc[qi * scs + j] = ((s0 + s1) + (s2 + s3)) * scale;
        }
      }
    }
  }
  __syncthreads();
  // per wave (query): max, exponentials (+0.0 past the last position, to a multiple of 16), the
  // in-order sum, p_j = e_j * inv
  float* const sw = sc + w * scs;
  float mx = -INFINITY;
  for (int j = lane; j < nw; j += 64) mx = fmaxf(mx, sw[j]);
  mx = wave_max(mx);
  const int n16 = (nw + 15) & ~15;
  for (int j = lane; j < n16; j += 64) sw[j] = j < nw ? elm_expf(sw[j] - mx) : 0.f;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  float sum = 0.f;
  for (int g0 = 0; g0 < n16; g0 += 256) sum = ordered_sum256(sw + g0, min(16, (n16 - g0) >> 4), sum);
  const float inv = 1.0f / sum;
  __builtin_amdgcn_wave_barrier();
  for (int j = lane; j < n16; j += 64) sw[j] = sw[j] * inv;
  wait_vm<0>();  // this wave's value rows
  __syncthreads();  // every value row in LDS; every wave's p_j written

  // o_i = 0, o_i += p_j * v_j[i] in increasing j (lane i), value chunks of R rows alternating
  // between the two buffers, the next chunk in flight while the waves add the current one
  float acc = 0.f;
  for (int c0 = 0, ci = 0; c0 < nmax; c0 += R, ++ci) {
    const float* const cur = (ci & 1) ? kb : vb;
    const int nx = c0 + R;
    if (nx < nmax) dma_rows(vh, vnew, nx, min(R, nmax - nx), (ci & 1) ? vb : kb, false);
    const int m = max(min(R, nw - c0), 0);  // this query's positions in the chunk
    acc = ordered_dot_col<R / 16>(sw + c0, cur + lane, m, acc);
    if (nx < nmax) {
      wait_vm<0>();
      __syncthreads();  // every wave is done with this chunk; the next one has landed
    }
  }
  if (w < nq) {
    out[(int64_t)tw * qd + h * HD + lane] = acc;
    if (xq) {
      // the next GEMM's activation fragments: lanes 0-31 hold block 2h of token tw, lanes 32-63
      // block 2h + 1; scale = amax / 127 and edgelm's rounding, as act_quant_frag_kernel
      float a = fmaxf(0.f, fabsf(acc));
#pragma unroll
      for (int k = 1; k < 32; k <<= 1) a = fmaxf(a, __shfl_xor(a, k, 64));
      const float scl = a / 127.0f;
      int qv;
      elm_q8_group<1>(&acc, scl == 0.f ? 1.f : scl, &qv);
      const int b = 2 * h + (lane >> 5), e = lane & 31;
      xq[elm_frag_offset(tw, b, e >> 4, 2 * n_heads) + (e & 15)] = (int8_t)qv;
      if (e == 0) xd[(int64_t)b * Tpad + tw] = scl;
    }
  }
}

// ---------------------------------------------------------------- EMBED

// y[t][k] = dequantize_row(table, tokens[t])[k] read from the repacked weight layout:
//   q8: float(q) * s_row;  q4: float(nibble - 8) * s_group
__global__ __launch_bounds__(256) void embed_kernel(const int32_t* __restrict__ tok, int64_t total,
                                                    const uint8_t* __restrict__ data,
                                                    const float* __restrict__ scales, int dtype, int64_t cols,
                                                    int64_t nb, int H, int64_t rows, float* __restrict__ y) {
  // every argument into scalar registers first, in one batch of loads (as the attention kernels)
  asm volatile("" ::"s"(tok), "s"(total), "s"(data), "s"(scales), "s"(dtype), "s"(cols), "s"(nb), "s"(H), "s"(rows),
               "s"(y), "s"(gridDim.x));
  for (int64_t idx = blockIdx.x * 256ll + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    const int64_t t = idx / cols, k = idx - t * cols;
    // ids are the caller's to check (edgelm checks them on the host); clamping keeps a bad id in bounds
    const int64_t row = min(max((int64_t)tok[t], (int64_t)0), rows - 1), b = k >> 5;
    const int j = (int)(k & 31);
    const int64_t it = item_index(row, b, nb, H);
    float v;
    if (dtype == WQ8) {
      v = (float)(int8_t)data[it * 32 + j] * scales[row];
    } else {
      const uint8_t byte = data[it * 16 + (j & 15)];
      const int nib = j < 16 ? (byte & 0x0F) : (byte >> 4);
      v = (float)(nib - 8) * scales[it];
    }
    y[idx] = v;
  }
}

// ---------------------------------------------------------------- fill

// dst[0 .. bytes) = value, 4 bytes per store where aligned (a kernel rather than hipMemsetAsync, so
// that callers may capture it in a HIP graph)
__global__ __launch_bounds__(256) void fill_kernel(uint8_t* __restrict__ dst, size_t bytes, uint32_t v4) {
  const size_t head = (4 - (reinterpret_cast<uintptr_t>(dst) & 3)) & 3;
  const size_t h = head < bytes ? head : bytes;
  const size_t words = (bytes - h) / 4;
  const size_t stride = (size_t)gridDim.x * 256;
  const size_t i0 = blockIdx.x * (size_t)256 + threadIdx.x;
  uint32_t* d4 = reinterpret_cast<uint32_t*>(dst + h);
  for (size_t i = i0; i < words; i += stride) d4[i] = v4;
  if (i0 < h) dst[i0] = (uint8_t)v4;
  const size_t tail = h + words * 4;
  if (i0 < bytes - tail) dst[tail + i0] = (uint8_t)v4;
}

// ---------------------------------------------------------------- read-bandwidth ceiling

// Reads every 16-byte word of src[0, n16) once (grid-stride, kReadSweepUnroll loads in flight per
// thread) and folds them by XOR; each wave stores its fold to sink[block * 4 + wave], so no load
// can be dropped. A measured ceiling for the GEMVs' read streams.
constexpr int kReadSweepBlocks = 2048, kReadSweepUnroll = 8;
__global__ __launch_bounds__(256) void read_sweep_kernel(const uint4* __restrict__ src, size_t n16,
                                                         uint32_t* __restrict__ sink) {
  const size_t stride = (size_t)gridDim.x * 256;
  size_t i = blockIdx.x * (size_t)256 + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (kReadSweepUnroll - 1) * stride < n16; i += kReadSweepUnroll * stride) {
    uint4 v[kReadSweepUnroll];
#pragma unroll
    for (int u = 0; u < kReadSweepUnroll; ++u) v[u] = src[i + u * stride];
#pragma unroll
    for (int u = 0; u < kReadSweepUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += stride) {
    const uint4 v = src[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, off, 64);
  if ((threadIdx.x & 63) == 0) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = acc;
}

}  // namespace

// ---------------------------------------------------------------- greedy sampling
//
// argmax (tokenizer.cpp:187-189) is std::max_element: a scan keeping the first index whose value
// no later value exceeds under IEEE <. So ties keep the earlier index (-0 and +0 tie), a NaN after
// index 0 is never taken, and a NaN at index 0 is kept (nothing compares greater). As a reduction:
// candidates are the non-NaN values plus index 0 if it is NaN (which beats everything); the
// larger value wins and equal values go to the smaller index. That order is total, so the
// per-thread scans and the tree below may combine in any order.
struct ArgBest {
  float v;
  int i;  // -1: no candidate
};

__device__ __forceinline__ ArgBest arg_pick(ArgBest a, ArgBest b) {
  if (a.i < 0) return b;
  if (b.i < 0) return a;
  const bool an = a.i == 0 && a.v != a.v, bn = b.i == 0 && b.v != b.v;  // NaN at index 0
  if (an || bn) return an ? a : b;
  if (a.v > b.v) return a;
  if (b.v > a.v) return b;
  return a.i < b.i ? a : b;
}

// one workgroup of kArgThreads per row
constexpr int kArgThreads = 1024;
constexpr int kArgVF = 12;  // float4 per thread per batch: 49,152 logits in one batch

__global__ __launch_bounds__(kArgThreads) void argmax_kernel(const float* __restrict__ x, int64_t n,
                                                             int32_t* __restrict__ out) {
  __shared__ float sv[kArgThreads / 64];
  __shared__ int si[kArgThreads / 64];
  const float* row = x + (int64_t)blockIdx.x * n;
  const int tid = threadIdx.x;
  // Each thread scans its values in increasing index: the first candidate is its first value that
  // is not NaN (or index 0 whatever it is), then only a strictly greater value replaces it. That
  // keeps the first index among equal values, lets a NaN at index 0 stand (nothing compares
  // greater than it) and skips every later NaN: max_element's answer for the thread's values.
  float bv = 0.f;
  int bi = -1;
  auto scan = [&](float v, int j) {
    const bool take = bi < 0 ? (v == v || j == 0) : v > bv;
    bv = take ? v : bv;
    bi = take ? j : bi;
  };
  const int64_t n4 = n >> 2;
  for (int64_t b0 = 0; b0 < n4; b0 += (int64_t)kArgThreads * kArgVF) {
    float4 v[kArgVF];  // every load of the batch in flight before the first compare
#pragma unroll
    for (int u = 0; u < kArgVF; ++u) {
      const float* p = row + 4 * min(b0 + tid + (int64_t)u * kArgThreads, n4 - 1);
      v[u] = make_float4(p[0], p[1], p[2], p[3]);
    }
#pragma unroll
    for (int u = 0; u < kArgVF; ++u) {
      const int64_t q = b0 + tid + (int64_t)u * kArgThreads;
      if (q < n4) {
        scan(v[u].x, (int)(4 * q));
        scan(v[u].y, (int)(4 * q + 1));
        scan(v[u].z, (int)(4 * q + 2));
        scan(v[u].w, (int)(4 * q + 3));
      }
    }
  }
  for (int64_t j = 4 * n4 + tid; j < n; j += kArgThreads) scan(row[j], (int)j);
  ArgBest best{bv, bi};
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const ArgBest o{__shfl_xor(best.v, off, 64), __shfl_xor(best.i, off, 64)};
    best = arg_pick(best, o);
  }
  const int wave = tid >> 6;
  if ((tid & 63) == 0) {
    sv[wave] = best.v;
    si[wave] = best.i;
  }
  __syncthreads();
  if (tid == 0) {
    ArgBest b{sv[0], si[0]};
    for (int w = 1; w < kArgThreads / 64; ++w) b = arg_pick(b, ArgBest{sv[w], si[w]});
    out[blockIdx.x] = b.i;  // n >= 1 and index 0 is always a candidate, so b.i >= 0
  }
}

// The argmax of one row over kArgPartMax workgroups at most: workgroup b scans the slice
// [b S, (b + 1) S) by argmax_kernel's rule (the first candidate: the slice's first value that is
// not NaN, or index 0; then only a strictly greater value) and posts its best; the last workgroup
// to post (a device-scope counter) merges the posts with arg_pick, which no order of merging
// changes, writes the index and clears the counter for the next launch. With `pos` given it also
// feeds a greedy decode step on the device: ring[*pos & ring_mask] = index, then *pos + 1.
namespace {

constexpr int kArgPartThreads = 256;
constexpr int kArgPartMax = 64;
constexpr int kArgPartVF = 4;  // float4 per thread: slices of 4096 values

__global__ __launch_bounds__(kArgPartThreads) void argmax_parts_kernel(const float* __restrict__ x, int n, int slice,
                                                                       float* __restrict__ post_v,
                                                                       int* __restrict__ post_i,
                                                                       unsigned* __restrict__ counter,
                                                                       int32_t* __restrict__ out, int32_t* __restrict__ pos,
                                                                       int32_t* __restrict__ ring, int ring_mask) {
  __shared__ float sv[kArgPartThreads / 64];
  __shared__ int si[kArgPartThreads / 64];
  __shared__ bool last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j0 = blockIdx.x * slice, j1 = min(n, j0 + slice);
  float bv = 0.f;
  int bi = -1;
  auto scan = [&](float v, int j) {
    const bool take = bi < 0 ? (v == v || j == 0) : v > bv;
    bv = take ? v : bv;
    bi = take ? j : bi;
  };
  // thread t takes float4 t, t + 256, ... of the slice (slices start on a multiple of 4), in
  // increasing index; every load out before the first compare
  const int q0 = j0 >> 2, nq = (j1 - j0) >> 2;
  if (nq > 0) {  // loads past the slice's last float4 repeat it
    float4 v[kArgPartVF];
#pragma unroll
    for (int u = 0; u < kArgPartVF; ++u) {
      const float* p = x + 4 * (q0 + min(tid + u * kArgPartThreads, nq - 1));
      v[u] = make_float4(p[0], p[1], p[2], p[3]);
    }
#pragma unroll
    for (int u = 0; u < kArgPartVF; ++u) {
      const int q = tid + u * kArgPartThreads;
      if (q < nq) {
        const int j = 4 * (q0 + q);
        scan(v[u].x, j);
        scan(v[u].y, j + 1);
        scan(v[u].z, j + 2);
        scan(v[u].w, j + 3);
      }
    }
  }
  for (int j = j0 + 4 * nq + tid; j < j1; j += kArgPartThreads) scan(x[j], j);  // the row's tail
  ArgBest best{bv, bi};
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) best = arg_pick(best, ArgBest{__shfl_xor(best.v, off, 64), __shfl_xor(best.i, off, 64)});
  if (lane == 0) {
    sv[wave] = best.v;
    si[wave] = best.i;
  }
  __syncthreads();
  if (tid == 0) {
    ArgBest b{sv[0], si[0]};
    for (int w = 1; w < kArgPartThreads / 64; ++w) b = arg_pick(b, ArgBest{sv[w], si[w]});
    post_v[blockIdx.x] = b.v;
    post_i[blockIdx.x] = b.i;
    __threadfence();  // the post is visible device-wide before the count says so
    last = atomicAdd(counter, 1u) == gridDim.x - 1;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();  // every other workgroup's post, as counted
  ArgBest b{0.f, -1};
  if (tid < (int)gridDim.x) b = ArgBest{post_v[tid], post_i[tid]};
  if (wave == 0) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) b = arg_pick(b, ArgBest{__shfl_xor(b.v, off, 64), __shfl_xor(b.i, off, 64)});
    if (lane == 0) {
      out[0] = b.i;  // n >= 1 and index 0 is always a candidate, so b.i >= 0
      if (pos) {
        const int p = pos[0];
        ring[p & ring_mask] = b.i;
        pos[0] = p + 1;
      }
      counter[0] = 0u;
    }
  }
}

}  // namespace

size_t argmax_parts_scratch_bytes() { return kArgPartMax * (sizeof(float) + sizeof(int)) + sizeof(unsigned); }

hipError_t launch_argmax_parts(const float* x, int64_t n, int32_t* out, int32_t* pos, int32_t* ring, int ring_mask,
                               void* scratch, hipStream_t s) {
  // slices of kArgPartThreads * kArgPartVF * 4 values at most, a multiple of 4, at most kArgPartMax of them
  const int64_t per = (int64_t)kArgPartThreads * kArgPartVF * 4;
  const int64_t parts = (n + per - 1) / per;
  if (n < 1 || parts > kArgPartMax) return hipErrorInvalidValue;
  const int slice = (int)((((n + parts - 1) / parts) + 3) & ~(int64_t)3);
  float* post_v = static_cast<float*>(scratch);
  int* post_i = reinterpret_cast<int*>(post_v + kArgPartMax);
  unsigned* counter = reinterpret_cast<unsigned*>(post_i + kArgPartMax);
  argmax_parts_kernel<<<(unsigned)((n + slice - 1) / slice), kArgPartThreads, 0, s>>>(
      x, (int)n, slice, post_v, post_i, counter, out, pos, ring, ring_mask);
  return hipGetLastError();
}

hipError_t launch_argmax(const float* x, int rows, int64_t n, int32_t* out, hipStream_t s) {
  argmax_kernel<<<rows, kArgThreads, 0, s>>>(x, n, out);
  return hipGetLastError();
}

hipError_t launch_fill(void* dst, int value, size_t bytes, hipStream_t s) {
  if (bytes == 0) return hipSuccess;
  const uint32_t b = (uint32_t)(value & 0xFF);
  const size_t blocks = (bytes / 4 + 255) / 256;
  fill_kernel<<<(unsigned)(blocks < 1 ? 1 : blocks < 8192 ? blocks : 8192), 256, 0, s>>>(
      static_cast<uint8_t*>(dst), bytes, b | (b << 8) | (b << 16) | (b << 24));
  return hipGetLastError();
}

size_t read_sweep_sink_bytes() { return (size_t)kReadSweepBlocks * 4 * sizeof(uint32_t); }

hipError_t launch_read_sweep(const void* src, size_t bytes, void* sink, hipStream_t s) {
  if (bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16) return hipErrorInvalidValue;
  read_sweep_kernel<<<kReadSweepBlocks, 256, 0, s>>>(static_cast<const uint4*>(src), bytes / 16,
                                                     static_cast<uint32_t*>(sink));
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const float* x, const float* w, float* y, int rows, int dim, float eps, hipStream_t s) {
  if (dim < 1 || dim > 256 * 4 * kNormVF) return hipErrorInvalidValue;
  const size_t rowlen = ((size_t)(dim >> 2) + 31) & ~(size_t)31;
  rmsnorm_kernel<<<rows, 256, (4 * rowlen + 4) * sizeof(float), s>>>(x, w, y, dim, eps);
  return hipGetLastError();
}

// attention_decode64_kernel: two row buffers, the scores (a multiple of 256), q and the step's key
size_t attention_decode_lds_bytes(int n_cap) {
  return ((size_t)2 * kDecRows * 64 + (size_t)((n_cap + 255) & ~255) + 128) * sizeof(float);
}

size_t attention_lds_bytes(int hd, int n_max) {
  const size_t hdp = (size_t)((hd + 3) & ~3);
  return (2 * hdp + (size_t)((n_max + 63) & ~63) + (size_t)attn_chunk_pos(hd) * hd) * sizeof(float);
}

// attention_kernel with its score rows in global memory (GS): LDS holds q, the fused key and a chunk
static size_t attention_gs_lds_bytes(int hd) {
  return (2 * (size_t)((hd + 3) & ~3) + (size_t)attn_chunk_pos(hd) * hd) * sizeof(float);
}

size_t attention_global_score_bytes(int T, int pos0, bool pos_dev, int n_heads, int hd, int max_ctx) {
  const int n_cap = pos_dev ? max_ctx : pos0 + T;
  if (attention_lds_bytes(hd, n_cap) <= kMaxAttnLds) return 0;
  return (size_t)T * n_heads * (size_t)((n_cap + 63) & ~63) * sizeof(float);
}

// the attention kernels keep a whole score row (and a chunk of values) in LDS: allow them up to kMaxAttnLds
bool raise_lds_limit() {
  const void* kernels[] = {(const void*)attention_kernel<64, false>, (const void*)attention_kernel<0, false>,
                           (const void*)attention_kernel<64, true>, (const void*)attention_kernel<0, true>,
                           (const void*)attention_prefill_kernel, (const void*)attention_decode64_kernel,
                           (const void*)attention_prefill64_kernel};
  for (const void* k : kernels) {
    hipFuncAttributes fa;
    if (hipFuncGetAttributes(&fa, k) != hipSuccess || fa.sharedSizeBytes + kMaxAttnLds > kMaxLds) return false;
    if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxAttnLds) != hipSuccess) return false;
  }
  return true;
}

hipError_t launch_attention(const float* q, const float* k, const float* v, float* out, int T, int pos0,
                            const int* pos_dev, int n_heads, int n_kv, int hd, float* kc, float* vc, int max_ctx,
                            const float* rcos, const float* rsin, hipStream_t s, int8_t* xq, float* xd, int Tpad,
                            bool* quantized, float* gscores) {
  if (quantized) *quantized = false;
  // with the position in device memory the score buffer covers the whole cache
  const int n_cap = pos_dev ? max_ctx : pos0 + T;  // score slots
  // one token, and chunks on the head-size-64 prefill kernel: the append runs inside the attention
  // kernel; other chunks append every key first
  const bool fuse = T == 1;
  const size_t lds_pf = ((size_t)kAttnQ * hd + (size_t)kAttnQ * ((n_cap + 63) & ~63) + (size_t)kAttnPVPos * hd) * 4;
  const size_t lds_pf64 = ((size_t)2 * kPfRows * 64 + (size_t)kAttnQ * ((n_cap + 255) & ~255) + (size_t)kAttnQ * 64) * 4;
  const bool pf64 = !fuse && hd == 64 && lds_pf64 <= kMaxAttnLds && !pos_dev;
  if (!fuse && !pf64) {
    kv_append_kernel<<<T * n_kv, 64, 0, s>>>(k, v, kc, vc, pos0, pos_dev, n_kv, hd, max_ctx, rcos, rsin);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const float* kn = fuse ? k : nullptr;
  const float* vn = fuse ? v : nullptr;
  static const bool lds_ok = raise_lds_limit();  // once per process (the attribute holds for the kernel)
  if (!lds_ok) return hipErrorInvalidValue;
  if (pf64) {
    const int ngr = (T + kAttnQ - 1) / kAttnQ;
    const bool quant = xq && xd && quantized;
    attention_prefill64_kernel<<<dim3(ngr, n_heads / n_kv, n_kv), 256, lds_pf64, s>>>(
        q, out, kc, vc, pos0, T, n_heads / n_kv, n_kv, max_ctx, n_cap, rcos, rsin, quant ? xq : nullptr,
        quant ? xd : nullptr, Tpad, k, v);
    const hipError_t e = hipGetLastError();
    if (e == hipSuccess && quant) *quantized = true;
    return e;
  }
  if (!fuse && hd == 64 && lds_pf <= kMaxAttnLds) {
    const int ngr = (T + kAttnQ - 1) / kAttnQ;
    const bool quant = xq && xd && quantized;
    attention_prefill_kernel<<<n_heads * ngr, 256, lds_pf, s>>>(q, out, kc, vc, pos0, T, n_heads, n_kv, max_ctx, n_cap,
                                                                rcos, rsin, quant ? xq : nullptr,
                                                                quant ? xd : nullptr, Tpad);
    const hipError_t e = hipGetLastError();
    if (e == hipSuccess && quant) *quantized = true;
    return e;
  }
  const bool in_lds = attention_lds_bytes(hd, n_cap) <= kMaxAttnLds;
  if (!in_lds && !gscores) return hipErrorInvalidValue;  // a score row past LDS needs the global rows
  const size_t lds_gs = attention_gs_lds_bytes(hd), lds = attention_lds_bytes(hd, n_cap);
  if (fuse && hd == 64 && attention_decode_lds_bytes(n_cap) <= kMaxAttnLds)
    attention_decode64_kernel<<<dim3(n_kv, n_heads / n_kv), 256, attention_decode_lds_bytes(n_cap), s>>>(
        q, out, kc, vc, pos0, pos_dev, n_heads / n_kv, n_kv, max_ctx, n_cap, rcos, rsin, k, v);
  else if (hd == 64 && in_lds)
    attention_kernel<64, false><<<T * n_heads, kAttnThreads, lds, s>>>(
        q, out, kc, vc, pos0, pos_dev, n_heads, n_kv, hd, max_ctx, n_cap, rcos, rsin, kn, vn, nullptr);
  else if (hd == 64)
    attention_kernel<64, true><<<T * n_heads, kAttnThreads, lds_gs, s>>>(
        q, out, kc, vc, pos0, pos_dev, n_heads, n_kv, hd, max_ctx, n_cap, rcos, rsin, kn, vn, gscores);
  else if (in_lds)
    attention_kernel<0, false><<<T * n_heads, kAttnThreads, lds, s>>>(
        q, out, kc, vc, pos0, pos_dev, n_heads, n_kv, hd, max_ctx, n_cap, rcos, rsin, kn, vn, nullptr);
  else
    attention_kernel<0, true><<<T * n_heads, kAttnThreads, lds_gs, s>>>(
        q, out, kc, vc, pos0, pos_dev, n_heads, n_kv, hd, max_ctx, n_cap, rcos, rsin, kn, vn, gscores);
  return hipGetLastError();
}

hipError_t launch_embed(const int32_t* tok, int T, const DevWeight& w, float* y, hipStream_t s) {
  const int64_t total = (int64_t)T * w.cols;
  const int64_t blocks = (total + 255) / 256;
  embed_kernel<<<(unsigned)(blocks < 4096 ? blocks : 4096), 256, 0, s>>>(tok, total, w.data, w.scales, w.dtype, w.cols,
                                                                         w.nb, w.H, w.rows, y);
  return hipGetLastError();
}

}  // namespace elmh

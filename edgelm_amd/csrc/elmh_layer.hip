// The non-matmul ops of a transformer layer on the device, so that a whole layer stays in HBM
// between consecutive ops: token embedding, RMSNORM, and attention with the rotary embedding and
// the KV-cache append fused in. Every float operation happens in the order of edgelm's cpu
// backend (x86 scalar path, no FMA contraction), so results are bit-identical to it:
//   rmsnorm   kernels_cpu.cpp:326-335 with dot_f32_scalar (kernels_cpu.cpp:30-43)
//   attention kernels_cpu.cpp:417-488 (append with rotated keys, then one task per (token, head))
//   embed     dequantize_row (model.cpp:192-218) of the token's row, EMBED (backends.cpp, reference)
#include <hip/hip_runtime.h>

#include "elm_expf.h"
#include "elmh_internal.hpp"

namespace elmh {
namespace {

// ---------------------------------------------------------------- RMSNORM
//
// One workgroup per row. The row goes to LDS; lanes 0-3 then run dot_f32_scalar's four strided
// accumulators s_k = sum of x[i]^2 over i = k (mod 4) in increasing i (the tail past the last
// multiple of 4 goes into s0), and ss = (s0 + s1) + (s2 + s3); inv = 1 / sqrt(ss / dim + eps);
// y[i] = (x[i] * inv) * w[i].
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                      float* __restrict__ y, int dim, float eps) {
  extern __shared__ float xs[];
  __shared__ float part[4];
  const int64_t r = blockIdx.x;
  const float* xr = x + r * dim;
  for (int i = threadIdx.x; i < dim; i += 256) xs[i] = xr[i];
  __syncthreads();
  if (threadIdx.x < 4) {
    const int k = threadIdx.x, m4 = dim & ~3;
    float s = 0.f;
#pragma unroll 8
    for (int i = k; i < m4; i += 4) s = s + xs[i] * xs[i];
    if (k == 0)
      for (int i = m4; i < dim; ++i) s = s + xs[i] * xs[i];
    part[k] = s;
  }
  __syncthreads();
  const float ss = (part[0] + part[1]) + (part[2] + part[3]);
  const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
  float* yr = y + r * dim;
  for (int i = threadIdx.x; i < dim; i += 256) yr[i] = (xs[i] * inv) * w[i];
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
// cache [kv_head][pos][hd]. One workgroup per (token, kv head).
__global__ __launch_bounds__(64) void kv_append_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                       float* __restrict__ kc, float* __restrict__ vc, int pos0,
                                                       int n_kv, int hd, int max_ctx, const float* __restrict__ rcos,
                                                       const float* __restrict__ rsin) {
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

// Step 2 of cpu::attention: one wave per (query token t, head h) over positions 0 .. pos0 + t.
//   q rotated into LDS; sc[j] = dot_f32(q, k_j) * scale in parallel over j; mx = max sc;
//   e_j = expf(sc[j] - mx); sum = e_0 + e_1 + ... in order (one lane); inv = 1 / sum;
//   lane i: o_i = 0, then o_i += (e_j * inv) * v_j[i] in increasing j.
// LDS: hd floats of q, then pos0 + T floats of scores.
__global__ __launch_bounds__(64) void attention_kernel(const float* __restrict__ q, float* __restrict__ out,
                                                       const float* __restrict__ kc, const float* __restrict__ vc,
                                                       int pos0, int n_heads, int n_kv, int hd, int max_ctx,
                                                       const float* __restrict__ rcos, const float* __restrict__ rsin) {
  extern __shared__ float lds[];
  float* qb = lds;
  float* sc = lds + ((hd + 3) & ~3);
  __shared__ float inv_s;
  const int lane = threadIdx.x;
  const int t = blockIdx.x / n_heads, h = blockIdx.x - t * n_heads, pos = pos0 + t, h2 = hd / 2, n = pos + 1;
  const int qd = n_heads * hd, grp = n_heads / n_kv;
  const float* qs = q + (int64_t)t * qd + h * hd;
  if (rcos) {
    const float* c = rcos + (int64_t)pos * h2;
    const float* s = rsin + (int64_t)pos * h2;
    for (int i = lane; i < h2; i += 64) {
      qb[i] = qs[i] * c[i] - qs[i + h2] * s[i];
      qb[i + h2] = qs[i + h2] * c[i] + qs[i] * s[i];
    }
  } else {
    for (int i = lane; i < hd; i += 64) qb[i] = qs[i];
  }
  __syncthreads();
  const float* kh = kc + (int64_t)(h / grp) * max_ctx * hd;
  const float* vh = vc + (int64_t)(h / grp) * max_ctx * hd;
  const float scale = 1.0f / sqrtf((float)hd);
  float mx = -INFINITY;
  for (int j = lane; j < n; j += 64) {
    const float s = dot4(qb, kh + (int64_t)j * hd, hd) * scale;
    sc[j] = s;
    mx = fmaxf(mx, s);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  for (int j = lane; j < n; j += 64) sc[j] = elm_expf(sc[j] - mx);
  __syncthreads();
  if (lane == 0) {
    float sum = 0.f;
#pragma unroll 8
    for (int j = 0; j < n; ++j) sum = sum + sc[j];
    inv_s = 1.0f / sum;
  }
  __syncthreads();
  const float inv = inv_s;
  float* o = out + (int64_t)t * qd + h * hd;
  for (int i = lane; i < hd; i += 64) {
    float acc = 0.f;
#pragma unroll 4
    for (int j = 0; j < n; ++j) acc = acc + (sc[j] * inv) * vh[(int64_t)j * hd + i];
    o[i] = acc;
  }
}

// ---------------------------------------------------------------- EMBED

// y[t][k] = dequantize_row(table, tokens[t])[k] read from the repacked weight layout:
//   q8: float(q) * s_row;  q4: float(nibble - 8) * s_group, s_group = (stored s/16) * 16
__global__ __launch_bounds__(256) void embed_kernel(const int32_t* __restrict__ tok, int64_t total,
                                                    const uint8_t* __restrict__ data,
                                                    const float* __restrict__ scales, int dtype, int64_t cols,
                                                    int64_t nb, int H, float* __restrict__ y) {
  for (int64_t idx = blockIdx.x * 256ll + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    const int64_t t = idx / cols, k = idx - t * cols;
    const int64_t row = tok[t], b = k >> 5;
    const int j = (int)(k & 31);
    const int64_t it = item_index(row, b, nb, H);
    float v;
    if (dtype == WQ8) {
      v = (float)(int8_t)data[it * 32 + j] * scales[row];
    } else {
      const uint8_t byte = data[it * 16 + (j & 15)];
      const int nib = j < 16 ? (byte & 0x0F) : (byte >> 4);
      v = (float)(nib - 8) * (scales[it] * 16.0f);
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

}  // namespace

hipError_t launch_fill(void* dst, int value, size_t bytes, hipStream_t s) {
  if (bytes == 0) return hipSuccess;
  const uint32_t b = (uint32_t)(value & 0xFF);
  const size_t blocks = (bytes / 4 + 255) / 256;
  fill_kernel<<<(unsigned)(blocks < 1 ? 1 : blocks < 8192 ? blocks : 8192), 256, 0, s>>>(
      static_cast<uint8_t*>(dst), bytes, b | (b << 8) | (b << 16) | (b << 24));
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const float* x, const float* w, float* y, int rows, int dim, float eps, hipStream_t s) {
  rmsnorm_kernel<<<rows, 256, (size_t)dim * sizeof(float), s>>>(x, w, y, dim, eps);
  return hipGetLastError();
}

size_t attention_lds_bytes(int hd, int n_max) { return ((size_t)((hd + 3) & ~3) + (size_t)n_max) * sizeof(float); }

hipError_t launch_attention(const float* q, const float* k, const float* v, float* out, int T, int pos0, int n_heads,
                            int n_kv, int hd, float* kc, float* vc, int max_ctx, const float* rcos, const float* rsin,
                            hipStream_t s) {
  kv_append_kernel<<<T * n_kv, 64, 0, s>>>(k, v, kc, vc, pos0, n_kv, hd, max_ctx, rcos, rsin);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  attention_kernel<<<T * n_heads, 64, attention_lds_bytes(hd, pos0 + T), s>>>(q, out, kc, vc, pos0, n_heads, n_kv, hd,
                                                                              max_ctx, rcos, rsin);
  return hipGetLastError();
}

hipError_t launch_embed(const int32_t* tok, int T, const DevWeight& w, float* y, hipStream_t s) {
  const int64_t total = (int64_t)T * w.cols;
  const int64_t blocks = (total + 255) / 256;
  embed_kernel<<<(unsigned)(blocks < 4096 ? blocks : 4096), 256, 0, s>>>(tok, total, w.data, w.scales, w.dtype, w.cols,
                                                                         w.nb, w.H, y);
  return hipGetLastError();
}

}  // namespace elmh

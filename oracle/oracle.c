/*
 * TEST INFRASTRUCTURE ONLY — CPU oracle for the quantized-matmul hot path (see oracle.h).
 * A restatement in C of edgelm's scalar algorithms; every function cites the reference
 * file:line it follows. Built by oracle/Makefile with -O2 -ffp-contract=off (no -march), so
 * every float operation rounds exactly where the reference's x86-64 scalar path rounds.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define ACT_BLOCK 32 /* kActBlock, include/edgelm/kernels.hpp:38 */
#define ROW_BLOCK 16 /* kRowBlock, include/edgelm/kernels.hpp:75 */

/* std::max / std::min as the reference calls them (a < b ? b : a) for finite operands. */
static float fmax_std(float a, float b) { return (a < b) ? b : a; }
static float fmin_std(float a, float b) { return (b < a) ? b : a; }

float orc_round_away(float v) { return copysignf(floorf(fabsf(v) + 0.5f), v); } /* model.cpp:63 */

/* model.cpp:150-163: per-row symmetric int8, scale = amax/127, round half away from zero. */
void orc_quantize_q8(const float* w, int64_t n, int64_t k, int8_t* out, float* scales) {
  for (int64_t r = 0; r < n; ++r) {
    const float* row = w + r * k;
    float amax = 0.f;
    for (int64_t i = 0; i < k; ++i) amax = fmax_std(amax, fabsf(row[i]));
    const float s = amax / 127.0f;
    const float safe = s == 0.f ? 1.f : s;
    scales[r] = s;
    for (int64_t i = 0; i < k; ++i) {
      const float q = orc_round_away(row[i] / safe);
      out[r * k + i] = (int8_t)fmin_std(127.f, fmax_std(-127.f, q));
    }
  }
}

/* model.cpp:165-190: group-32 int4; d = x[first argmax |x|] / -8; q in [-8,7] stored as q+8;
 * byte j of a group = element j (low nibble) | element j+16 (high nibble). */
void orc_quantize_q4(const float* w, int64_t n, int64_t k, uint8_t* out, float* scales) {
  const int G = 32;
  for (int64_t r = 0; r < n; ++r) {
    for (int64_t g = 0; g < k / G; ++g) {
      const float* x = w + r * k + g * G;
      int best = 0;
      float amax = fabsf(x[0]);
      for (int i = 1; i < G; ++i) {
        const float a = fabsf(x[i]);
        if (a > amax) {
          amax = a;
          best = i;
        }
      }
      const float d = x[best] / -8.0f;
      const float safe = d == 0.f ? 1.f : d;
      scales[r * (k / G) + g] = d;
      uint8_t* o = out + r * (k / 2) + g * (G / 2);
      for (int i = 0; i < G / 2; ++i) {
        const uint8_t lo = (uint8_t)(fmin_std(7.f, fmax_std(-8.f, orc_round_away(x[i] / safe))) + 8);
        const uint8_t hi = (uint8_t)(fmin_std(7.f, fmax_std(-8.f, orc_round_away(x[i + G / 2] / safe))) + 8);
        o[i] = (uint8_t)(lo | (hi << 4));
      }
    }
  }
}

/* model.cpp:192-218 */
void orc_dequantize_row(const orc_weight* w, int64_t row, float* out) {
  const int64_t k = w->cols;
  if (w->dtype == ORC_F32) {
    memcpy(out, (const float*)w->data + row * k, (size_t)k * sizeof(float));
  } else if (w->dtype == ORC_Q8) {
    const int8_t* q = (const int8_t*)w->data + row * k;
    const float s = w->scales[row];
    for (int64_t i = 0; i < k; ++i) out[i] = (float)q[i] * s;
  } else {
    const uint8_t* q = (const uint8_t*)w->data + row * (k / 2);
    const float* s = w->scales + row * (k / 32);
    for (int64_t g = 0; g < k / 32; ++g)
      for (int i = 0; i < 16; ++i) {
        const uint8_t b = q[g * 16 + i];
        out[g * 32 + i] = (float)((int)(b & 0x0F) - 8) * s[g];
        out[g * 32 + 16 + i] = (float)((int)(b >> 4) - 8) * s[g];
      }
  }
}

/* kernels_ref.cpp:23-37: per 32-block amax, d = amax/127, q = clamp(copysign(floor(|x/safe|+.5)),+-127) */
void orc_quantize_act_row(const float* x, int64_t k, int8_t* q, float* d) {
  for (int64_t b = 0; b < k / ACT_BLOCK; ++b) {
    const float* xb = x + b * ACT_BLOCK;
    float amax = 0.f;
    for (int i = 0; i < ACT_BLOCK; ++i) amax = fmax_std(amax, fabsf(xb[i]));
    const float s = amax / 127.0f;
    const float safe = s == 0.f ? 1.f : s;
    d[b] = s;
    for (int i = 0; i < ACT_BLOCK; ++i) {
      const float v = xb[i] / safe;
      const float r = copysignf(floorf(fabsf(v) + 0.5f), v);
      q[b * ACT_BLOCK + i] = (int8_t)fmin_std(127.f, fmax_std(-127.f, r));
    }
  }
}

/* kernels.hpp:46-48 */
int orc_act_quant_applies(const orc_weight* w) {
  return (w->dtype == ORC_Q8 || w->dtype == ORC_Q4) && w->cols % ACT_BLOCK == 0;
}

/* kernels_cpu.cpp:292 (silu1) and kernels_ref.cpp:146-148: libm expf, IEEE divide. */
float orc_silu(float v) { return v / (1.0f + expf(-v)); }

/* ------------------------------------------------------------------ reference backend */

/* kernels_ref.cpp:58-80 */
void orc_ref_matmul(const float* x, int T, const orc_weight* w, float* y, const float* residual, int act_quant) {
  const int64_t N = w->rows, K = w->cols;
  float* xf = NULL;
  if (act_quant && orc_act_quant_applies(w)) {
    xf = (float*)malloc(sizeof(float) * (size_t)T * (size_t)K);
    int8_t* q = (int8_t*)malloc((size_t)K);
    float* d = (float*)malloc(sizeof(float) * (size_t)(K / ACT_BLOCK));
    for (int t = 0; t < T; ++t) {
      orc_quantize_act_row(x + t * K, K, q, d);
      for (int64_t i = 0; i < K; ++i) xf[t * K + i] = (float)q[i] * d[i / ACT_BLOCK];
    }
    free(q);
    free(d);
    x = xf;
  }
  float* row = (float*)malloc(sizeof(float) * (size_t)K);
  for (int64_t n = 0; n < N; ++n) {
    orc_dequantize_row(w, n, row);
    for (int t = 0; t < T; ++t) {
      float acc = 0.f;
      for (int64_t k = 0; k < K; ++k) acc += x[t * K + k] * row[k];
      y[t * N + n] = residual ? residual[t * N + n] + acc : acc;
    }
  }
  free(row);
  free(xf);
}

/* kernels_ref.cpp:153-160 */
void orc_ref_swiglu(const float* x, int T, const orc_weight* wg, const orc_weight* wu, float* y, int act_quant) {
  const int64_t n = (int64_t)T * wg->rows;
  float* g = (float*)malloc(sizeof(float) * (size_t)n);
  float* u = (float*)malloc(sizeof(float) * (size_t)n);
  orc_ref_matmul(x, T, wg, g, NULL, act_quant);
  orc_ref_matmul(x, T, wu, u, NULL, act_quant);
  for (int64_t i = 0; i < n; ++i) g[i] = g[i] / (1.0f + expf(-g[i])); /* kernels_ref.cpp:146-148 */
  for (int64_t i = 0; i < n; ++i) y[i] = g[i] * u[i];                 /* kernels_ref.cpp:149-151 */
  free(g);
  free(u);
}

/* ------------------------------------------------------------------ cpu backend, x86 scalar */

/* kernels_cpu.cpp:32-43: four interleaved accumulators, tail into the first. */
static float dot_f32_scalar(const float* a, const float* b, int64_t k) {
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  int64_t i = 0;
  for (; i + 4 <= k; i += 4) {
    s0 += a[i] * b[i];
    s1 += a[i + 1] * b[i + 1];
    s2 += a[i + 2] * b[i + 2];
    s3 += a[i + 3] * b[i + 3];
  }
  for (; i < k; ++i) s0 += a[i] * b[i];
  return (s0 + s1) + (s2 + s3);
}

/* kernels_cpu.cpp:45-71 (scalar part; unscaled) */
static float dot_q8(const float* x, const int8_t* w, int64_t k) {
  int64_t i = 0;
  float s = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  for (; i + 4 <= k; i += 4) {
    s += x[i] * (float)w[i];
    s1 += x[i + 1] * (float)w[i + 1];
    s2 += x[i + 2] * (float)w[i + 2];
    s3 += x[i + 3] * (float)w[i + 3];
  }
  for (; i < k; ++i) s += x[i] * (float)w[i];
  return (s + s1) + (s2 + s3);
}

/* kernels_cpu.cpp:73-112 (scalar part; scaled per group) */
static float dot_q4(const float* x, const uint8_t* w, const float* scales, int64_t k) {
  const int64_t groups = k / 32;
  float s = 0.f;
  for (int64_t g = 0; g < groups; ++g) {
    float g0 = 0.f, g1 = 0.f;
    for (int i = 0; i < 16; ++i) {
      const uint8_t b = w[g * 16 + i];
      g0 += x[g * 32 + i] * (float)((int)(b & 0x0F) - 8);
      g1 += x[g * 32 + 16 + i] * (float)((int)(b >> 4) - 8);
    }
    s += (g0 + g1) * scales[g];
  }
  return s;
}

/* kernels_cpu.cpp:114-123 */
static float dot_row(const float* x, const orc_weight* w, int64_t r) {
  const int64_t K = w->cols;
  if (w->dtype == ORC_F32) return dot_f32_scalar(x, (const float*)w->data + r * K, K);
  if (w->dtype == ORC_Q8) return dot_q8(x, (const int8_t*)w->data + r * K, K) * w->scales[r];
  return dot_q4(x, (const uint8_t*)w->data + r * (K / 2), w->scales + r * (K / 32), K);
}

/* kernels_cpu.cpp:138-205, scalar branches: int32 per 32-block, f32 mul then add. */
static float dot_a8_1(const int8_t* xq, const float* xd, int64_t K, const orc_weight* w, int64_t r) {
  const int64_t nb = K / ACT_BLOCK;
  float acc = 0.f;
  if (w->dtype == ORC_Q8) {
    const int8_t* wr = (const int8_t*)w->data + r * K;
    for (int64_t b = 0; b < nb; ++b) {
      int32_t s = 0;
      for (int i = 0; i < 32; ++i) s += (int32_t)wr[b * 32 + i] * xq[b * 32 + i];
      acc += (float)s * xd[b];
    }
    return acc * w->scales[r];
  }
  const uint8_t* wr = (const uint8_t*)w->data + r * (K / 2);
  const float* ws = w->scales + r * nb;
  for (int64_t g = 0; g < nb; ++g) {
    int32_t s = 0;
    for (int i = 0; i < 16; ++i) {
      const uint8_t b = wr[g * 16 + i];
      s += ((int32_t)(b & 0x0F) - 8) * xq[g * 32 + i] + ((int32_t)(b >> 4) - 8) * xq[g * 32 + 16 + i];
    }
    acc += (float)s * (ws[g] * xd[g]);
  }
  return acc;
}

/* kernels_cpu.cpp:207-220: out[t*ldo] for all T tokens (the 4-token variant computes each token
 * with the same scalar arithmetic, so one token at a time is equivalent). */
static void row_a8(const int8_t* q, const float* d, int T, const orc_weight* w, int64_t r, float* out, int64_t ldo) {
  const int64_t K = w->cols, nb = K / ACT_BLOCK;
  for (int t = 0; t < T; ++t) out[t * ldo] = dot_a8_1(q + t * K, d + t * nb, K, w, r);
}

/* kernels_cpu.cpp:254-283 (scalar part) */
static void gemm_f32(const float* x, int T, const float* w, int R, int64_t K, float* y, int64_t ldy, const float* res) {
  for (int t0 = 0; t0 < T; ++t0)
    for (int j = 0; j < R; ++j) {
      const int64_t idx = (int64_t)t0 * ldy + j;
      y[idx] = (res ? res[idx] : 0.f) + dot_f32_scalar(x + (int64_t)t0 * K, w + (int64_t)j * K, K);
    }
}

/* kernels_cpu.cpp:285-290 */
static const float* weight_tile(const orc_weight* w, int64_t r0, int nr, float* buf) {
  if (w->dtype == ORC_F32) return (const float*)w->data + r0 * w->cols;
  for (int i = 0; i < nr; ++i) orc_dequantize_row(w, r0 + i, buf + (int64_t)i * w->cols);
  return buf;
}

/* kernels_cpu.cpp:222-228 */
static void quantize_rows(const float* x, int T, int64_t K, int8_t* q, float* d) {
  for (int t = 0; t < T; ++t) orc_quantize_act_row(x + t * K, K, q + t * K, d + t * (K / ACT_BLOCK));
}

/* kernels_cpu.cpp:339-377 */
void orc_cpu_matmul(const float* x, int T, int n_targets, const orc_weight* w, float* const* y,
                    const float* const* residual, int act_quant) {
  int a8 = 0;
  if (act_quant)
    for (int i = 0; i < n_targets; ++i) a8 |= orc_act_quant_applies(&w[i]);
  const int64_t K0 = w[0].cols;
  int8_t* aq_q = NULL;
  float* aq_d = NULL;
  if (a8) {
    aq_q = (int8_t*)malloc((size_t)T * (size_t)K0);
    aq_d = (float*)malloc(sizeof(float) * (size_t)T * (size_t)(K0 / ACT_BLOCK + 1));
    quantize_rows(x, T, K0, aq_q, aq_d);
  }
  int64_t maxk = 0;
  for (int i = 0; i < n_targets; ++i) maxk = w[i].cols > maxk ? w[i].cols : maxk;
  float* scratch = (float*)malloc(sizeof(float) * (size_t)(ROW_BLOCK * maxk + 16));
  for (int i = 0; i < n_targets; ++i) {
    const orc_weight* wt = &w[i];
    const int64_t N = wt->rows;
    const float* res = residual ? residual[i] : NULL;
    float* yi = y[i];
    for (int64_t r0 = 0; r0 < N; r0 += ROW_BLOCK) {
      const int nr = (int)((N - r0) < ROW_BLOCK ? (N - r0) : ROW_BLOCK);
      if (a8 && orc_act_quant_applies(wt)) {
        for (int64_t r = r0; r < r0 + nr; ++r) {
          row_a8(aq_q, aq_d, T, wt, r, yi + r, N);
          if (res)
            for (int t = 0; t < T; ++t) yi[t * N + r] += res[t * N + r];
        }
      } else if (T == 1) {
        for (int64_t r = r0; r < r0 + nr; ++r) yi[r] = (res ? res[r] : 0.f) + dot_row(x, wt, r);
      } else {
        const float* tile = weight_tile(wt, r0, nr, scratch);
        gemm_f32(x, T, tile, nr, wt->cols, yi + r0, N, res ? res + r0 : NULL);
      }
    }
  }
  free(scratch);
  free(aq_q);
  free(aq_d);
}

/* kernels_cpu.cpp:379-411 */
void orc_cpu_swiglu(const float* x, int T, const orc_weight* wg, const orc_weight* wu, float* y, int act_quant) {
  const int64_t N = wg->rows, K = wg->cols;
  const int a8 = act_quant && orc_act_quant_applies(wg) && orc_act_quant_applies(wu);
  int8_t* aq_q = NULL;
  float* aq_d = NULL;
  if (a8) {
    aq_q = (int8_t*)malloc((size_t)T * (size_t)K);
    aq_d = (float*)malloc(sizeof(float) * (size_t)T * (size_t)(K / ACT_BLOCK + 1));
    quantize_rows(x, T, K, aq_q, aq_d);
  }
  float* deq = (float*)malloc(sizeof(float) * (size_t)(ROW_BLOCK * K + 2 * (int64_t)T * ROW_BLOCK + 16));
  float* G = deq + ROW_BLOCK * K;
  float* U = G + (int64_t)T * ROW_BLOCK;
  for (int64_t r0 = 0; r0 < N; r0 += ROW_BLOCK) {
    const int nr = (int)((N - r0) < ROW_BLOCK ? (N - r0) : ROW_BLOCK);
    if (a8) {
      for (int j = 0; j < nr; ++j) {
        row_a8(aq_q, aq_d, T, wg, r0 + j, G + j, ROW_BLOCK);
        row_a8(aq_q, aq_d, T, wu, r0 + j, U + j, ROW_BLOCK);
      }
    } else if (T == 1) {
      for (int64_t r = r0; r < r0 + nr; ++r) y[r] = orc_silu(dot_row(x, wg, r)) * dot_row(x, wu, r);
      continue;
    } else {
      gemm_f32(x, T, weight_tile(wg, r0, nr, deq), nr, K, G, ROW_BLOCK, NULL);
      gemm_f32(x, T, weight_tile(wu, r0, nr, deq), nr, K, U, ROW_BLOCK, NULL);
    }
    for (int t = 0; t < T; ++t)
      for (int j = 0; j < nr; ++j) y[t * N + r0 + j] = orc_silu(G[t * ROW_BLOCK + j]) * U[t * ROW_BLOCK + j];
  }
  free(deq);
  free(aq_q);
  free(aq_d);
}

/* Brute-force int32 block sums (kernels_cpu.cpp:159-167 q8, 193-204 q4). */
void orc_block_sums(const int8_t* xq, int T, const orc_weight* w, int32_t* S) {
  const int64_t N = w->rows, K = w->cols, nb = K / ACT_BLOCK;
  for (int t = 0; t < T; ++t)
    for (int64_t n = 0; n < N; ++n)
      for (int64_t b = 0; b < nb; ++b) {
        int32_t s = 0;
        for (int i = 0; i < 32; ++i) {
          const int64_t k = b * 32 + i;
          int wq;
          if (w->dtype == ORC_Q8) {
            wq = ((const int8_t*)w->data)[n * K + k];
          } else {
            const uint8_t byte = ((const uint8_t*)w->data)[n * (K / 2) + b * 16 + (i & 15)];
            wq = (i < 16 ? (byte & 0x0F) : (byte >> 4)) - 8;
          }
          s += wq * xq[(int64_t)t * K + k];
        }
        S[((int64_t)t * N + n) * nb + b] = s;
      }
}

/* ------------------------------------------------------------------ per-token extension */

void orc_quantize_act_row_token(const float* x, int64_t k, int8_t* q, float* d) {
  float amax = 0.f;
  for (int64_t i = 0; i < k; ++i) amax = fmax_std(amax, fabsf(x[i]));
  const float s = amax / 127.0f;
  const float safe = s == 0.f ? 1.f : s;
  *d = s;
  for (int64_t i = 0; i < k; ++i) {
    const float v = x[i] / safe;
    const float r = copysignf(floorf(fabsf(v) + 0.5f), v);
    q[i] = (int8_t)fmin_std(127.f, fmax_std(-127.f, r));
  }
}

void orc_matmul_a8_token(const float* x, int T, const orc_weight* w, float* y, const float* residual) {
  const int64_t N = w->rows, K = w->cols, nb = K / ACT_BLOCK;
  int8_t* q = (int8_t*)malloc((size_t)K);
  for (int t = 0; t < T; ++t) {
    float d;
    orc_quantize_act_row_token(x + t * K, K, q, &d);
    for (int64_t n = 0; n < N; ++n) {
      float out;
      if (w->dtype == ORC_Q8) {
        const int8_t* wr = (const int8_t*)w->data + n * K;
        int32_t s = 0;
        for (int64_t k = 0; k < K; ++k) s += (int32_t)wr[k] * q[k];
        out = ((float)s * d) * w->scales[n];
      } else {
        const uint8_t* wr = (const uint8_t*)w->data + n * (K / 2);
        float acc = 0.f;
        for (int64_t g = 0; g < nb; ++g) {
          int32_t s = 0;
          for (int i = 0; i < 16; ++i) {
            const uint8_t b = wr[g * 16 + i];
            s += ((int32_t)(b & 0x0F) - 8) * q[g * 32 + i] + ((int32_t)(b >> 4) - 8) * q[g * 32 + 16 + i];
          }
          acc += (float)s * w->scales[n * nb + g];
        }
        out = acc * d;
      }
      y[t * N + n] = residual ? residual[t * N + n] + out : out;
    }
  }
  free(q);
}

/* ------------------------------------------------------------------ layer ops (cpu backend) */

/* kernels_ref.cpp:11-21: the RopeTable, computed in double, [pos][head_dim/2] */
void orc_rope_table(int head_dim, int max_pos, float theta, float* cos_out, float* sin_out) {
  const int half = head_dim / 2;
  for (int p = 0; p < max_pos; ++p)
    for (int i = 0; i < half; ++i) {
      const double inv = pow((double)theta, -2.0 * i / head_dim);
      const double a = p * inv;
      cos_out[(int64_t)p * half + i] = (float)cos(a);
      sin_out[(int64_t)p * half + i] = (float)sin(a);
    }
}

/* kernels_cpu.cpp:326-335 with dot_f32_scalar: inv = 1 / sqrt(dot(x, x) / dim + eps), y = x * inv * w */
void orc_rmsnorm(const float* x, const float* w, float* y, int rows, int dim, float eps) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * dim;
    const float inv = 1.0f / sqrtf(dot_f32_scalar(xr, xr, dim) / dim + eps);
    for (int i = 0; i < dim; ++i) y[r * dim + i] = xr[i] * inv * w[i];
  }
}

/* kernels_cpu.cpp:417-488 (serial): append this step's keys (rotated when rcos != NULL) and values
 * to the cache [n_kv][max_ctx][hd], then one task per (token, head). */
void orc_attention(const float* q, const float* k, const float* v, float* out, int T, int pos0, int n_heads, int n_kv,
                   int hd, float* kc, float* vc, int max_ctx, const float* rcos, const float* rsin) {
  const int h2 = hd / 2, kvd = n_kv * hd, qd = n_heads * hd, grp = n_heads / n_kv;
  const int64_t mc = max_ctx;
  for (int t = 0; t < T; ++t) {
    const int pos = pos0 + t;
    for (int h = 0; h < n_kv; ++h) {
      const float* ks = k + (int64_t)t * kvd + h * hd;
      float* kd = kc + (h * mc + pos) * hd;
      if (rcos) {
        const float* c = rcos + (int64_t)pos * h2;
        const float* sn = rsin + (int64_t)pos * h2;
        for (int i = 0; i < h2; ++i) {
          kd[i] = ks[i] * c[i] - ks[i + h2] * sn[i];
          kd[i + h2] = ks[i + h2] * c[i] + ks[i] * sn[i];
        }
      } else {
        memcpy(kd, ks, sizeof(float) * hd);
      }
      memcpy(vc + (h * mc + pos) * hd, v + (int64_t)t * kvd + h * hd, sizeof(float) * hd);
    }
  }
  const float scale = 1.0f / sqrtf((float)hd);
  float* qbuf = (float*)malloc(sizeof(float) * (size_t)hd);
  float* sc = (float*)malloc(sizeof(float) * (size_t)(pos0 + T));
  for (int64_t idx = 0; idx < (int64_t)T * n_heads; ++idx) {
    const int t = (int)(idx / n_heads), h = (int)(idx % n_heads), pos = pos0 + t;
    const float* qs = q + (int64_t)t * qd + h * hd;
    if (rcos) {
      const float* c = rcos + (int64_t)pos * h2;
      const float* sn = rsin + (int64_t)pos * h2;
      for (int i = 0; i < h2; ++i) {
        qbuf[i] = qs[i] * c[i] - qs[i + h2] * sn[i];
        qbuf[i + h2] = qs[i + h2] * c[i] + qs[i] * sn[i];
      }
      qs = qbuf;
    }
    const float* kh = kc + (int64_t)(h / grp) * mc * hd;
    const float* vh = vc + (int64_t)(h / grp) * mc * hd;
    const int n = pos + 1;
    float mx = -INFINITY;
    for (int j = 0; j < n; ++j) {
      sc[j] = dot_f32_scalar(qs, kh + (int64_t)j * hd, hd) * scale;
      mx = fmax_std(mx, sc[j]);
    }
    float sum = 0.f;
    for (int j = 0; j < n; ++j) sum += (sc[j] = expf(sc[j] - mx));
    const float inv = 1.0f / sum;
    float* o = out + (int64_t)t * qd + h * hd;
    for (int i = 0; i < hd; ++i) o[i] = 0.f;
    for (int j = 0; j < n; ++j) {
      const float p = sc[j] * inv;
      const float* vj = vh + (int64_t)j * hd;
      for (int i = 0; i < hd; ++i) o[i] += p * vj[i];
    }
  }
  free(qbuf);
  free(sc);
}

/* argmax (tokenizer.cpp:187-189): std::max_element over [x, x + n) keeps the current best unless
 * best < candidate, scanning forward; restated as that scan. */
int32_t orc_argmax(const float* x, int64_t n) {
  int64_t best = 0;
  for (int64_t i = 1; i < n; ++i)
    if (x[best] < x[i]) best = i;
  return (int32_t)best;
}

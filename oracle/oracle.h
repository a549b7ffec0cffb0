/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle for the quantized-matmul hot path.
 *
 * A plain-C restatement of edgelm's own algorithms for this path (reference at
 * adarsh-sgh/edgelm, cited as file:line below). Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only as the checker or the CPU baseline:
 * the product (edgelm_amd/) never links, loads or falls back to it.
 *
 * Every function is pinned against the reference's own C++ compiled from its sources into
 * oracle/_ref (see oracle/Makefile), against closed forms (quantizer error bounds, max
 * element -> +-127 / -8, zero rows) and against brute force (integer block sums).
 * Compile with -ffp-contract=off and no -march so float order matches the reference's
 * x86-64 scalar path (kernels_cpu.cpp:15-20 selects it where NEON is absent).
 */
#ifndef EDGELM_ORACLE_H
#define EDGELM_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype values match edgelm's DType (include/edgelm/graph.hpp:17). */
enum { ORC_F32 = 0, ORC_Q8 = 1, ORC_Q4 = 2 };

typedef struct {
  int dtype;            /* ORC_F32 / ORC_Q8 / ORC_Q4 */
  int64_t rows, cols;   /* N, K */
  const void* data;     /* f32 [N,K] | int8 [N,K] | u8 [N,K/2] */
  const float* scales;  /* q8: [N]; q4: [N, K/32]; f32: NULL */
} orc_weight;

/* model.cpp:63 */
float orc_round_away(float v);
/* model.cpp:150-163 */
void orc_quantize_q8(const float* w, int64_t n, int64_t k, int8_t* out, float* scales);
/* model.cpp:165-190 */
void orc_quantize_q4(const float* w, int64_t n, int64_t k, uint8_t* out, float* scales);
/* model.cpp:192-218 */
void orc_dequantize_row(const orc_weight* w, int64_t row, float* out);
/* kernels_ref.cpp:23-37 */
void orc_quantize_act_row(const float* x, int64_t k, int8_t* q, float* d);
/* kernels.hpp:46-48 */
int orc_act_quant_applies(const orc_weight* w);
/* kernels_cpu.cpp:292 / kernels_ref.cpp:146-148: v / (1 + exp(-v)) */
float orc_silu(float v);

/* kernels_ref.cpp:58-80 (the reference backend's matmul) */
void orc_ref_matmul(const float* x, int T, const orc_weight* w, float* y, const float* residual, int act_quant);
/* kernels_ref.cpp:153-160 */
void orc_ref_swiglu(const float* x, int T, const orc_weight* wg, const orc_weight* wu, float* y, int act_quant);

/* kernels_cpu.cpp:339-377 on the x86 scalar path, serial (results do not depend on threads,
 * test_e2e.cpp:77-99). y[i] / residual[i] belong to target i; residual may be NULL. */
void orc_cpu_matmul(const float* x, int T, int n_targets, const orc_weight* w, float* const* y,
                    const float* const* residual, int act_quant);
/* kernels_cpu.cpp:379-411 on the x86 scalar path */
void orc_cpu_swiglu(const float* x, int T, const orc_weight* wg, const orc_weight* wu, float* y, int act_quant);

/* int32 per-(token, row, 32-block) sums S[t][n][b] = sum_i wq * xq (kernels_cpu.cpp:159-167,
 * 193-204), brute force. xq is [T, K] as produced by orc_quantize_act_row. */
void orc_block_sums(const int8_t* xq, int T, const orc_weight* w, int32_t* S);

/* ---- per-token activation scale: an extension with no counterpart in edgelm ----
 * One scale per row: d = amax(row)/127, q = clamp(round_away(x/safe), +-127) (the same
 * rounding as quantize_act_row, over the whole row instead of 32-blocks). */
void orc_quantize_act_row_token(const float* x, int64_t k, int8_t* q, float* d);
/* y = (res? res : 0) + out, with
 *   q8: out = ((float)S * d_t) * ws[n], S = sum over all K (int32)
 *   q4: out = (sum_b (float)S_b * ws[n,b]) * d_t, sequential over b (mul, add) */
void orc_matmul_a8_token(const float* x, int T, const orc_weight* w, float* y, const float* residual);

/* kernels_ref.cpp:11-21: RopeTable cos/sin [max_pos][head_dim/2], computed in double */
void orc_rope_table(int head_dim, int max_pos, float theta, float* cos_out, float* sin_out);
/* kernels_cpu.cpp:326-335 (cpu::rmsnorm, x86 scalar dot_f32) */
void orc_rmsnorm(const float* x, const float* w, float* y, int rows, int dim, float eps);
/* kernels_cpu.cpp:417-488 (cpu::attention, serial); rcos/rsin NULL: no rotary embedding */
void orc_attention(const float* q, const float* k, const float* v, float* out, int T, int pos0, int n_heads, int n_kv,
                   int hd, float* kc, float* vc, int max_ctx, const float* rcos, const float* rsin);

/* argmax (tokenizer.cpp:187-189): std::max_element's scan, the first index whose value no later
 * value exceeds under IEEE <. */
int32_t orc_argmax(const float* x, int64_t n);
#ifdef __cplusplus
}
#endif
#endif

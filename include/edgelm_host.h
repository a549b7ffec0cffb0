/*
 * C API of the edgelm_amd host library (libedgelm_host.so): the C++17 restatement of the edgelm
 * host pieces the hot path needs around it, for callers that are not C++ (tests, bench.py).
 */
#ifndef EDGELM_HOST_H
#define EDGELM_HOST_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Load-time quantizers, bit-identical to edgelm's quantize_q8 (model.cpp:150-163) and
 * quantize_q4 (model.cpp:165-190); rows are split over `threads` host threads. Return 0, or -1
 * without writing anything for a bad shape (q4: K not a positive multiple of 32, as edgelm's
 * EDGELM_CHECK refuses) or a null pointer. */
int elm_quantize_q8(const float* w, int64_t n, int64_t k, int8_t* out, float* scales, int threads);
int elm_quantize_q4(const float* w, int64_t n, int64_t k, uint8_t* out, float* scales, int threads);

/* ---- models and sessions (edgelm's Model / Session, reference runtime.hpp:17-67) ----
 * Every call returns 0 / a handle on success; on failure -1 / NULL and elm_last_error() says why. */
typedef struct elm_model elm_model;
typedef struct elm_session elm_session;

const char* elm_last_error(void);

elm_model* elm_model_load(const char* path);
void elm_model_free(elm_model* m);
/* vocab, dim, hidden, n_layers, n_heads, n_kv_heads, head_dim, max_seq, weight dtype, tied */
int elm_model_config(const elm_model* m, int* out10);
/* Fusion statistics of the model's graph: swiglu, shared_input, residual, rope, ops_before, ops_after. */
int elm_model_fusion(const elm_model* m, int* out6);
/* Memory plan for T tokens / L logit rows (fused or not): writes arena, naive bytes; returns 1 if
 * plan_is_valid, 0 if not, -1 on error. */
int elm_model_plan(const elm_model* m, int fuse, int T, int L, int64_t* arena_bytes, int64_t* naive_bytes);
/* Partition the (fused) graph with a comma-separated backend preference ("hip" is planned without a
 * device); writes describe_partitions into buf; returns the number of partitions. */
int elm_model_partition(const elm_model* m, const char* backends, int fuse, char* buf, int cap);

/* backends: comma-separated preference ("hip,cpu"); the reference backend is appended last. */
elm_session* elm_session_create(const elm_model* m, const char* backends, int threads, int max_ctx, int max_batch,
                                int all_logits, int act_quant, int fuse);
void elm_session_destroy(elm_session* s);
/* forward(tokens[n]); copies rows * vocab logits to out (rows = all_logits ? n : 1). */
int elm_session_forward(elm_session* s, const int32_t* tokens, int n, float* out);
/* prefill in max_batch chunks; copies the last chunk's logits rows to out. */
int elm_session_prefill(elm_session* s, const int32_t* tokens, int n, float* out);
int elm_session_reset(elm_session* s);
int elm_session_pos(const elm_session* s);
int elm_session_describe(const elm_session* s, char* buf, int cap);
/* edgelm's bench protocol (main.cpp:173-233) on one session: reset, prefill the prompt, argmax
 * (TTFT), then gen greedy decode steps. Writes prefill ms, TTFT ms, decode ms and the gen + 1
 * generated token ids (first one from the prefill). Each argmax is taken where the logits are
 * (Session::greedy: on the device when a hip backend writes them), so the first one is part of the
 * prefill's last step and prefill ms equals TTFT ms. */
int elm_session_generate(elm_session* s, const int32_t* prompt, int n_prompt, int gen, double* prefill_ms,
                         double* ttft_ms, double* decode_ms, int32_t* tokens_out);

#ifdef __cplusplus
}
#endif
#endif

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

/* ---- synthetic models: a seeded random-init Llama-shaped model written as an .elm file (the
 * unfused graph edgelm's exporter emits, tools/elm.py:105-161; edgelm's loader reads it). Weight
 * matrices are N(0, sd), the embedding N(0, embed_sd), norm vectors 1 + N(0, norm_sd); each row comes
 * from its own splitmix64 stream of (seed, tensor, row), so the file does not depend on `threads`. */
typedef struct {
  int32_t vocab, dim, hidden, n_layers, n_heads, n_kv_heads, head_dim, max_seq;
  float rope_theta, norm_eps;
  int32_t bos, eos, tied;
  int32_t weight_dtype; /* every weight matrix: 0 f32, 1 q8, 2 q4 */
  int32_t embed_dtype;  /* the embedding (and tied LM head); -1: weight_dtype */
  uint64_t seed;
  float sd, embed_sd, norm_sd;
  int32_t threads;
} elm_model_spec;
int elm_write_random_model(const char* path, const elm_model_spec* spec);

/* ---- models and sessions (edgelm's Model / Session, reference runtime.hpp:17-67) ----
 * Every call returns 0 / a handle on success; on failure -1 / NULL and elm_last_error() says why. */
typedef struct elm_model elm_model;
typedef struct elm_session elm_session;

const char* elm_last_error(void);

elm_model* elm_model_load(const char* path);
void elm_model_free(elm_model* m);
/* Model::convert_weights (edgelm model.cpp:220-251): quantize the f32 weight matrices to dtype 1 (q8)
 * or 2 (q4) in memory, byte-identical to edgelm's; 0 keeps an f32 model. */
int elm_model_convert(elm_model* m, int dtype, int threads);
/* Model::prefault: touch every page of the mapping. */
int elm_model_prefault(const elm_model* m);
/* Device image (the cached repacked layout of the load path): elm_model_write_device_image writes every
 * q8 / q4 weight in the hip delegate's HBM layout to `path` and returns how many it wrote;
 * elm_model_attach_device_image maps such a file and returns 1, so that sessions made afterwards upload
 * the weights from it, or 0 (nothing changed) when the file is missing or belongs to other weights. */
int elm_model_write_device_image(const elm_model* m, const char* path, int threads);
int elm_model_attach_device_image(elm_model* m, const char* path);
/* Copies weight `name`'s data and scales (either may be NULL) and returns its dtype, or -1 if there is
 * no such weight; rows/cols get its shape. For tests of the loader and of convert_weights. */
int elm_model_weight(const elm_model* m, const char* name, int64_t* rows, int64_t* cols, void* data, float* scales);
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
/* Session::greedy: forward n tokens and take the argmax of the last logits row (where the logits are). */
int elm_session_greedy(elm_session* s, const int32_t* tokens, int n, int32_t* next);
/* Session::greedy_steps: n greedy decode steps from token `first` (the same tokens as n greedy calls,
 * fed back on the device where the hip backend runs the whole graph); tokens gets all n. */
int elm_session_greedy_steps(elm_session* s, int32_t first, int n, int32_t* tokens);
/* bench.py's protocol on one session: reset, prefill the prompt and take its greedy token (TTFT), run
 * `warmup` untimed greedy decode steps, then time exactly `steps` more (decode_ms), both through
 * Session::greedy_steps: the clock stops once every step's token id is on the host. tokens_out
 * (optional) gets the 1 + warmup + steps greedy tokens. */
int elm_session_bench(elm_session* s, const int32_t* prompt, int n_prompt, int warmup, int steps, double* ttft_ms,
                      double* decode_ms, int32_t* tokens_out);
int elm_session_generate(elm_session* s, const int32_t* prompt, int n_prompt, int gen, double* prefill_ms,
                         double* ttft_ms, double* decode_ms, int32_t* tokens_out);

/* ---- test hooks: the host ops a partition leaves on the CPU, alone. flavor 0 reproduces edgelm's
 * reference backend (kernels_ref.cpp:11-21,41-57,82-151), 1 its cpu backend's x86 scalar path
 * (kernels_cpu.cpp:326-335,413-492); threads > 1 splits the cpu flavor's rows / (token, head) items
 * over a pool. The caches are [n_kv][max_ctx][head_dim]; the RoPE table covers max_ctx positions.
 * Return 0, or -1 with elm_last_error() (context overflow, position beyond the table). */
int elm_host_rope_table(int head_dim, int max_pos, float theta, float* cos_out, float* sin_out);
int elm_host_rmsnorm(const float* x, const float* w, float* y, int rows, int dim, float eps, int flavor, int threads);
int elm_host_attention(const float* q, const float* k, const float* v, float* out, int T, int pos0, int n_heads,
                       int n_kv, int head_dim, float* kc, float* vc, int max_ctx, int rope, float theta, int flavor,
                       int threads);
int elm_host_rope(const float* x, float* y, int T, int n_heads, int head_dim, int pos0, int max_pos, float theta);
/* op: 0 add, 1 mul, 2 silu (b unused) */
int elm_host_elementwise(int op, const float* a, const float* b, float* y, int64_t n);

#ifdef __cplusplus
}
#endif
#endif

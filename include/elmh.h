/*
 * elmh — C ABI of the MI355X quantized-matmul delegate for edgelm.
 *
 * This is the boundary a HIP backend inside edgelm binds: edgelm's Backend::supports/run
 * (include/edgelm/backend.hpp:30-36) for MATMUL, MATMUL_N, MATMUL_ADD and FFN_SWIGLU reach
 * the GPU only through these calls (edgelm_amd/host/hip_backend.cpp is that backend).
 * Plain C types only; every call returns an elmh_status and never throws; the message of
 * the last failure is available from elmh_last_error().
 *
 * Numerics (edgelm reference, adarsh-sgh/edgelm):
 *  - weights: q8 = int8 [N,K] + f32 scale per row; q4 = 16 bytes per 32-group (element j
 *    in the low nibble of byte j, element j+16 in the high nibble, value q+8) + f32 scale
 *    per (row, group) — the export layout of tools/elm.py:41-71 / model.cpp:150-190;
 *  - ELMH_ACT_INT8: each activation row is quantized per 32-element block exactly like
 *    quantize_act_row (kernels_ref.cpp:23-37); int32 block sums are exact and the f32
 *    result equals the cpu backend's scalar path (kernels_cpu.cpp:138-228) bit for bit
 *    in ELMH_EXACT mode;
 *  - ELMH_ACT_F32: f32 activations, same order of float operations as the scalar
 *    dot_q8 / dot_q4 (T == 1) and dequantize + dot_f32 (T > 1) paths
 *    (kernels_cpu.cpp:32-123, 254-290);
 *  - FFN_SWIGLU: y = silu(x.Wg^T) * (x.Wu^T), silu(v) = v / (1 + expf(-v))
 *    (kernels_cpu.cpp:292, 379-411).
 *
 * Threading: one HIP stream per context; a context is not thread-safe. Host-pointer entry
 * points are synchronous (outputs are in host memory on return, as Backend::run requires);
 * *_dev entry points take device pointers and are stream-ordered on the context's stream.
 */
#ifndef ELMH_H
#define ELMH_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  ELMH_OK = 0,
  ELMH_ERR_ARG = 1,          /* bad argument (shape, dtype, null pointer) */
  ELMH_ERR_HIP = 2,          /* a HIP runtime call failed */
  ELMH_ERR_NODEV = 3,        /* no usable gfx950 device */
  ELMH_ERR_UNSUPPORTED = 4,  /* valid request outside what the kernels implement */
  ELMH_ERR_OOM = 5
} elmh_status;

/* weight dtypes: the values of edgelm's DType (include/edgelm/graph.hpp:17) */
enum { ELMH_F32 = 0, ELMH_Q8 = 1, ELMH_Q4 = 2 };

/* activation handling */
enum {
  ELMH_ACT_F32 = 0,        /* Session act_quant = false (runtime.hpp:25) */
  ELMH_ACT_INT8 = 1,       /* act_quant = true: per-row x per-32-block int8 (kernels.hpp:38-48) */
  ELMH_ACT_INT8_TOKEN = 2  /* extension, no counterpart in edgelm: one int8 scale per row */
};

/* f32 rescale order of the int8 GEMM (T > 4) */
enum {
  ELMH_EXACT = 0, /* sequential multiply then add per 32-block: bit-identical to the cpu backend */
  ELMH_FAST = 1   /* fused multiply-add per 32-block: within 1e-6 relative, not bit-identical */
};

typedef struct elmh_ctx elmh_ctx;
typedef struct elmh_weight elmh_weight;

/* ---- context (replaces nothing in edgelm: the cpu backend needs no device state) ---- */
int elmh_device_count(int* count);
int elmh_create(int device, elmh_ctx** out);
void elmh_destroy(elmh_ctx* ctx);
/* Message of the last failed call on ctx (ctx may be NULL: last failure on this thread). */
const char* elmh_last_error(const elmh_ctx* ctx);
/* Name of the device architecture the context runs on (e.g. "gfx950"). */
const char* elmh_device_arch(const elmh_ctx* ctx);

/* ---- weights: one upload per edgelm weight Tensor (graph.hpp:33-45) ----
 * Copies data/scales (host pointers, edgelm's export layout) into HBM in the repacked layout;
 * the host buffers are not retained. K must be a multiple of 32 for q4. */
int elmh_upload_weight(elmh_ctx* ctx, int dtype, int64_t rows, int64_t cols, const void* data,
                       const float* scales, elmh_weight** out);
int elmh_free_weight(elmh_ctx* ctx, elmh_weight* w);
/* Device bytes held by the weight (data + scales, after padding). */
size_t elmh_weight_bytes(const elmh_weight* w);

/* ---- device images of weights (the cached repacked layout of the load path, model.cpp:94-116) ----
 * The layout a weight has in HBM: row tiles of H rows, [rows_pad/H][nb][H] items of 32 (q8) or 16 (q4)
 * bytes, scales q8 [rows_pad], q4 [rows_pad/H][nb][H]; rows_pad = rows rounded up to 64. H depends on
 * dtype and cols only. elmh_weight_layout gives H and the byte counts; elmh_repack_host builds the
 * layout from edgelm's export layout on the CPU (the same bytes the upload's device repack writes);
 * elmh_upload_weight_image uploads a weight already in that layout (no repack launch, no staging of
 * the export layout); elmh_download_weight_image copies one back. No counterpart in edgelm: they let
 * a host cache the repacked weights on disk next to the .elm file. */
int elmh_weight_layout(int dtype, int64_t rows, int64_t cols, int* H, size_t* data_bytes, size_t* scale_bytes);
int elmh_repack_host(int dtype, int64_t rows, int64_t cols, const void* data, const float* scales, void* out_data,
                     float* out_scales);
int elmh_upload_weight_image(elmh_ctx* ctx, int dtype, int64_t rows, int64_t cols, const void* data,
                             const float* scales, elmh_weight** out);
int elmh_download_weight_image(elmh_ctx* ctx, const elmh_weight* w, void* data, float* scales);

/* ---- MATMUL / MATMUL_N / MATMUL_ADD (cpu::matmul, kernels_cpu.cpp:339-377) ----
 * For each target i: y[i][T, N_i] = (residual[i] ? residual[i] : 0) + x[T, K] . W_i^T.
 * x is quantized once for all targets (int8 modes). residual may be NULL, or residual[i]
 * NULL for a target without one. Host pointers; synchronous. */
int elmh_matmul(elmh_ctx* ctx, const float* x, int T, int64_t K, int n_targets, elmh_weight* const* w,
                float* const* y, const float* const* residual, int act, int mode);

/* ---- FFN_SWIGLU (cpu::swiglu, kernels_cpu.cpp:379-411) ----
 * y[T, N] = silu(x . Wg^T) * (x . Wu^T). Host pointers; synchronous. */
int elmh_swiglu(elmh_ctx* ctx, const float* x, int T, int64_t K, const elmh_weight* wg, const elmh_weight* wu,
                float* y, int act, int mode);

/* ---- device-resident variants: same semantics, device pointers, asynchronous on the context
 * stream (no host synchronization; capturable in a HIP graph once scratch is reserved). */
int elmh_reserve(elmh_ctx* ctx, int max_T, int64_t max_K);
/* Counter of the context's scratch reallocations. A *_dev call whose shape needs more scratch than is
 * reserved reallocates it (outside capture) and bumps the counter; a HIP graph captured while the
 * counter had another value holds freed addresses and must be captured again before it is launched.
 * No counterpart in edgelm: for callers that replay graphs (this build's hip backend). */
uint64_t elmh_scratch_generation(const elmh_ctx* ctx);
int elmh_matmul_dev(elmh_ctx* ctx, const float* x, int T, int64_t K, int n_targets, elmh_weight* const* w,
                    float* const* y, const float* const* residual, int act, int mode);
int elmh_swiglu_dev(elmh_ctx* ctx, const float* x, int T, int64_t K, const elmh_weight* wg,
                    const elmh_weight* wu, float* y, int act, int mode);
/* elmh_matmul_dev with no device allocation. No counterpart in edgelm: it is for callers that cannot
 * allocate (code under HIP graph capture, serving loops that must not call hipMalloc). The same kernels
 * and the same results, bit for bit; the quantized activation goes to a fixed 8 MiB device array of the
 * library (one per GPU, held until the process ends) instead of context scratch, so nothing is
 * allocated or freed. Limit: the quantized activation must fit the array; int8 activations with more
 * tokens than the GEMV takes need round_up(T, 128) * K bytes plus the scales, e.g. T <= 512 at
 * K <= 14336; larger calls fail with ELMH_ERR_ARG before anything runs. Every call on one GPU shares that
 * GPU's array (each call writes all of it that it reads): calls that overlap on one GPU (two contexts,
 * or two streams, in flight at once) race. */
int elmh_matmul_noalloc_dev(elmh_ctx* ctx, const float* x, int T, int64_t K, int n_targets, elmh_weight* const* w,
                            float* const* y, const float* const* residual, int act, int mode);

/* ---- pre-quantized activations (the ActBuf of kernels.hpp:39-44, row-major) ----
 * elmh_quantize_act_dev writes q [T, K] int8, d [T, K/32] f32 and s [T, K/32] int32 block
 * sums of q; elmh_gemv_a8_dev runs the T <= 4 int8 GEMV of MATMUL/MATMUL_ADD on them
 * (row_a8 with a shared ActBuf, kernels_cpu.cpp:207-220). */
int elmh_quantize_act_dev(elmh_ctx* ctx, const float* x, int T, int64_t K, int8_t* q, float* d, int32_t* s);
int elmh_gemv_a8_dev(elmh_ctx* ctx, const int8_t* q, const float* d, const int32_t* s, int T, int64_t K,
                     int n_targets, elmh_weight* const* w, float* const* y, const float* const* residual);
/* FFN_SWIGLU (int8 activations, exact mode) whose output row also comes back quantized for the next
 * int8 GEMV: y as elmh_swiglu_dev(x, T, K, wg, wu, y, ELMH_ACT_INT8, ELMH_EXACT) writes it, and q / d / s
 * as elmh_quantize_act_dev(y, T, N, q, d, s) then writes them (N = rows of wg, a multiple of 32), bit for
 * bit. The pair FFN_SWIGLU -> MATMUL_ADD down of a layer (passes.cpp:100-104) quantizes h once between
 * them (cpu::matmul's quantize_act_row of its input, kernels_cpu.cpp:339-377); where the streaming
 * GEMV runs the SwiGLU (one token, long weights), each workgroup owns whole 32-blocks of h and
 * quantizes them in its epilogue, so no quantizer launch runs; elsewhere the call launches it after
 * the SwiGLU. Pass q / d / s to elmh_gemv_a8_dev for the down projection. */
int elmh_swiglu_quant_dev(elmh_ctx* ctx, const float* x, int T, int64_t K, const elmh_weight* wg,
                          const elmh_weight* wu, float* y, int8_t* q, float* d, int32_t* s);

/* ---- the rest of a layer on the device (device pointers, asynchronous on the context stream) ----
 * Same float operations in the same order as edgelm's cpu backend, so results are bit-identical.
 *
 * EMBED (the reference backend's EMBED = dequantize_row per token, model.cpp:192-218):
 * y[t, :] = dequantize_row(table, tokens[t]) for a q8 or q4 table uploaded with
 * elmh_upload_weight; token ids must lie in [0, rows) (the caller checks, as edgelm does). */
int elmh_embed_dev(elmh_ctx* ctx, const int32_t* tokens, int T, const elmh_weight* table, float* y);
/* RMSNORM (cpu::rmsnorm, kernels_cpu.cpp:326-335): y = x * (1 / sqrt(dot_f32(x, x) / dim + eps)) * w
 * per row, dot_f32 in the four-accumulator order of dot_f32_scalar (kernels_cpu.cpp:30-43);
 * dim <= 8192. */
int elmh_rmsnorm_dev(elmh_ctx* ctx, const float* x, const float* w, float* y, int rows, int dim, float eps);
/* RMSNORM followed by the matmul or SwiGLU that consumes it, as one call: the same results as
 * elmh_rmsnorm_dev into a buffer and then elmh_matmul_dev / elmh_swiglu_dev on it (bit for bit),
 * for the edgelm op pairs RMSNORM -> MATMUL_N and RMSNORM -> FFN_SWIGLU of a layer
 * (passes.cpp:72-81,100-104; cpu::rmsnorm kernels_cpu.cpp:326-335). With int8 activations on
 * rows short enough for the workgroup-quantizing GEMV (T <= 4, K <= 2048) each workgroup
 * normalizes the rows itself and the normalized activation never goes to memory; on the
 * block-scale GEMM path (K <= 2048) one launch normalizes and quantizes the rows into the GEMM's
 * operand; otherwise the normalized rows go to a scratch buffer (reserved by elmh_reserve)
 * first. K <= 8192. */
int elmh_rmsnorm_matmul_dev(elmh_ctx* ctx, const float* x, const float* norm_w, float eps, int T, int64_t K,
                            int n_targets, elmh_weight* const* w, float* const* y, const float* const* residual,
                            int act, int mode);
int elmh_rmsnorm_swiglu_dev(elmh_ctx* ctx, const float* x, const float* norm_w, float eps, int T, int64_t K,
                            const elmh_weight* wg, const elmh_weight* wu, float* y, int act, int mode);
/* A layer's FFN pair as one call: FFN_SWIGLU of x (RMSNORM'd first when norm_w is given, as
 * elmh_rmsnorm_swiglu_dev) into h [T, N] (N = rows of wg), then MATMUL of h by wd into y [T, rows of
 * wd], plus res when given (MATMUL_ADD). The same results as elmh_rmsnorm_swiglu_dev /
 * elmh_swiglu_dev into h and then elmh_matmul_dev on h, bit for bit, h included: the op pair
 * FFN_SWIGLU -> MATMUL_ADD down of edgelm's fused layer (passes.cpp:100-104), the down projection
 * quantizing its input h once (cpu::matmul's quantize_act_row, kernels_cpu.cpp:339-377). With int8
 * activations at one token on the streaming GEMV (long rows) the SwiGLU launch quantizes h itself
 * (elmh_swiglu_quant_dev) and the down projection takes it pre-quantized, so no quantizer launch runs
 * between them; elmh_ffn_fused(ctx) returns 1 if the last call took that path, 0 otherwise. */
int elmh_ffn_dev(elmh_ctx* ctx, const float* x, const float* norm_w, float eps, int T, int64_t K,
                 const elmh_weight* wg, const elmh_weight* wu, float* h, elmh_weight* wd, float* y, const float* res,
                 int act, int mode);
int elmh_ffn_fused(const elmh_ctx* ctx);
/* ATTENTION (cpu::attention, kernels_cpu.cpp:417-488; AttnArgs, kernels.hpp:28-36): appends this
 * step's keys (rotated when rope_cos/rope_sin, the RopeTable's [pos][head_dim/2] arrays, are given)
 * and values to the cache [n_kv][max_ctx][head_dim] at positions pos0 .. pos0+T-1, then
 * out[t, h] = softmax over positions 0 .. pos0+t of (rotated q . k_j) / sqrt(head_dim), applied to v.
 * q [T, n_heads*head_dim], k/v [T, n_kv*head_dim]. */
int elmh_attention_dev(elmh_ctx* ctx, const float* q, const float* k, const float* v, float* out, int T, int pos0,
                       int n_heads, int n_kv, int head_dim, float* k_cache, float* v_cache, int max_ctx,
                       const float* rope_cos, const float* rope_sin);
/* ATTENTION followed by the MATMUL or MATMUL_ADD that consumes its output (a layer's o projection,
 * MATMUL_ADD after fuse_residual, passes.cpp:88-110; cpu::attention kernels_cpu.cpp:417-488), as
 * one call: the same results as elmh_attention_dev into out and then elmh_matmul_dev(out, T,
 * n_heads*head_dim, one target w -> y, residual res or NULL), bit for bit; out is written as
 * well. Where the chunk attention kernel (T > 1, head_dim 64) and the block-scale GEMM (int8
 * activations, too many rows for the GEMV) both apply, the attention kernel also writes its
 * output as the GEMM's quantized operand, so no quantizer launch runs in between. The GEMM then
 * also multiplies the token slots T .. round_up(T, 128) - 1 of that operand, which hold whatever an
 * earlier call left there: their results are never stored, and every stored output depends only on
 * its own token's slot. elmh_attention_matmul_fused(ctx) returns 1 if the last call took that path,
 * else 0 (no counterpart in edgelm: it lets a test tell the two paths apart). */
int elmh_attention_matmul_fused(const elmh_ctx* ctx);
int elmh_attention_matmul_dev(elmh_ctx* ctx, const float* q, const float* k, const float* v, float* out, int T,
                              int pos0, int n_heads, int n_kv, int head_dim, float* k_cache, float* v_cache,
                              int max_ctx, const float* rope_cos, const float* rope_sin, elmh_weight* w, float* y,
                              const float* res, int act, int mode);
/* One decode token (T = 1) of elmh_attention_dev with its position pos0 read from device memory
 * (*pos_dev, in [0, max_ctx)), so that a decode step captured in a HIP graph replays at every
 * position. No counterpart in edgelm: it serves callers that replay graphs (this build's hip
 * backend). The caller keeps *pos_dev within the cache and the rope table. */
int elmh_attention_step_dev(elmh_ctx* ctx, const float* q, const float* k, const float* v, float* out,
                            const int32_t* pos_dev, int n_heads, int n_kv, int head_dim, float* k_cache, float* v_cache,
                            int max_ctx, const float* rope_cos, const float* rope_sin);

/* 1 if elmh_attention_step_dev runs this head size with a cache of max_ctx positions, else 0. Every
 * context length runs, as in edgelm's attention: score rows longer than a workgroup's LDS holds (about
 * 20K positions at head size 64) live in a device buffer the context allocates on the first such call
 * (T * n_heads rows of the positions in use, or of max_ctx for elmh_attention_step_dev), with the same
 * float operations in the same order; a graph captured before that buffer grows must be captured again
 * (elmh_scratch_generation). No counterpart in edgelm. */
int elmh_attention_step_supported(int head_dim, int max_ctx);

/* Greedy sampling: argmax (tokenizer.cpp:187-189, std::max_element) of each row of x [rows, n]
 * (device pointers) into out [rows] (device int32): the first index of the largest value under
 * IEEE <, so NaNs after index 0 are never chosen and a NaN at index 0 is. Lets a caller take the
 * next token without copying the logits off the device. n >= 1. */
int elmh_argmax_dev(elmh_ctx* ctx, const float* x, int rows, int64_t n, int32_t* out);

/* One greedy decode step's tail on the device: *out = the argmax of the row x [n] (as
 * elmh_argmax_dev), then ring[*pos_dev & (ring_len - 1)] = that index and *pos_dev += 1, so that the
 * next step (its EMBED reading *out, its attention reading *pos_dev) follows with no host copy and the
 * host collects the token ids from ring later. ring_len is a power of two; n <= 262144. No counterpart
 * in edgelm: it is the device side of this build's greedy-steps hook (Session::greedy_steps). Calls on
 * one context run in stream order (they share a small counter in the context). */
int elmh_argmax_step_dev(elmh_ctx* ctx, const float* x, int64_t n, int32_t* out, int32_t* pos_dev, int32_t* ring,
                         int ring_len);

/* ---- test hooks ----
 * quantize_act_row on the device (host pointers; q [T,K], d [T,K/32]). */
int elmh_quantize_act(elmh_ctx* ctx, const float* x, int T, int64_t K, int8_t* q, float* d);
/* Exact int32 block sums S[t][n][b] = sum_i wq * xq over 32-block b (host pointers;
 * xq [T,K] int8 row-major; S [T, N, K/32]). */
int elmh_block_sums(elmh_ctx* ctx, const int8_t* xq, int T, const elmh_weight* w, int32_t* S);

/* ---- device memory, stream and timing plumbing for callers without a runtime of their own ---- */
int elmh_malloc(elmh_ctx* ctx, size_t bytes, void** dptr);
int elmh_free(elmh_ctx* ctx, void* dptr);
int elmh_memcpy_h2d(elmh_ctx* ctx, void* dst, const void* src, size_t bytes);
int elmh_memcpy_d2h(elmh_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Pinned host memory and stream-ordered copies, for a caller that moves activations between its
 * host arena and the device at every op (edgelm's Session hands backends host pointers op by op,
 * runtime.cpp:66-76): staged through pinned memory, an op's uploads, kernels and downloads are
 * enqueued together and waited for once (elmh_synchronize). An async copy returns once enqueued;
 * its host buffer must stay untouched, and its destination unread, until elmh_synchronize. No
 * counterpart in edgelm. */
int elmh_host_alloc(elmh_ctx* ctx, size_t bytes, void** ptr);
int elmh_host_free(elmh_ctx* ctx, void* ptr);
int elmh_memcpy_h2d_async(elmh_ctx* ctx, void* dst, const void* src, size_t bytes);
int elmh_memcpy_d2h_async(elmh_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Device fill (a kernel, so it may be captured in a HIP graph) and device-to-device copy; both
 * asynchronous on the context stream. LAST_ROWS (backends.cpp, reference) is one such copy. */
int elmh_memset_dev(elmh_ctx* ctx, void* dst, int value, size_t bytes);
int elmh_memcpy_d2d(elmh_ctx* ctx, void* dst, const void* src, size_t bytes);
int elmh_synchronize(elmh_ctx* ctx);
void* elmh_stream(elmh_ctx* ctx); /* the context's hipStream_t */
/* Measurement hook, no counterpart in edgelm: reads every 16-byte word of src[0, bytes) once (src and
 * bytes 16-byte aligned) and folds them into sink (elmh_read_sweep_sink_bytes() of device memory),
 * asynchronously on the context stream. Timed over a buffer far larger than the 256 MB Infinity
 * Cache it is the read ceiling of HBM; repeated over a buffer that stays in that cache (larger than
 * the L2s), the cache's; the benchmark reports the GEMVs against both. */
size_t elmh_read_sweep_sink_bytes(void);
int elmh_read_sweep_dev(elmh_ctx* ctx, const void* src, size_t bytes, void* sink);
/* Measurement hook, no counterpart in edgelm: the ceiling that edgelm's per-32-block activation scales
 * (kernels_cpu.cpp:159-167, 193-204: one f32 rescale of every block's int32 sum, multiply and add rounded
 * separately) put on an int8 MFMA GEMM, measured without memory traffic. `blocks` workgroups of four
 * waves each run `iters` 32-deep blocks: two v_mfma_i32_32x32x32_i8 per block (two 32 x 32 output tiles,
 * as a wave of the ring GEMM) and, by mode, no rescale (0: the sums accumulate in the MFMA, the per-token
 * form), the q8 rescale (1) or the q4 rescale (2) of the block's sums. Each thread writes one float to
 * sink (at least blocks * 1 KiB).
 * Asynchronous on the context stream. */
int elmh_rescale_ceiling_dev(elmh_ctx* ctx, int mode, int blocks, int iters, float* sink, size_t sink_bytes);
/* Events on the context stream: record, then elapsed milliseconds between two records. */
int elmh_event_create(elmh_ctx* ctx, void** ev);
int elmh_event_destroy(elmh_ctx* ctx, void* ev);
int elmh_event_record(elmh_ctx* ctx, void* ev);
int elmh_event_elapsed(elmh_ctx* ctx, void* start, void* stop, float* ms);
/* HIP graph capture of the context stream (launch-bound inner loops). */
int elmh_graph_begin(elmh_ctx* ctx);
int elmh_graph_end(elmh_ctx* ctx, void** graph_exec);
int elmh_graph_launch(elmh_ctx* ctx, void* graph_exec);
int elmh_graph_destroy(elmh_ctx* ctx, void* graph_exec);

#ifdef __cplusplus
}
#endif
#endif /* ELMH_H */

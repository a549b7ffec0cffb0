// Internal structures shared by the HIP kernels (elmh_kernels.hip) and the C-ABI layer
// (elmh_api.cpp). Not part of the public interface (include/elmh.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace elmh {

constexpr int kBlock = 32;       // activation block / q4 group (edgelm kActBlock, kernels.hpp:38)
constexpr int kMaxTargets = 4;   // weights per kernel launch (MATMUL_N with more is split)
constexpr int kGemvThreads = 256;
// Streaming GEMV: producer waves plus, for rows of more than kStreamFoldWaveBlocks blocks, one
// wave whose lanes fold (token, row) pairs while the weights stream (seven producer waves and two
// weight batches in flight per wave there; four producer waves and four batches otherwise).
constexpr int kStreamFoldLanes = 64;
constexpr int kStreamFoldWaveBlocks = 256;
constexpr int kStreamWavesShort = 4;
constexpr int kStreamWavesLong = 7;
inline int stream_producers(int nb) {
  return 64 * (nb > kStreamFoldWaveBlocks ? kStreamWavesLong : kStreamWavesShort);
}
// The streaming GEMV can also take f32 activations and quantize them in each workgroup: every
// producer thread holds up to 4 * kStreamQinPasses values (passes of 16). Only for rows without
// the fold wave (K <= 8192): every workgroup reads and rounds the whole activation, which at the
// 8B down GEMV's K = 14336 (57 KB of f32 per workgroup) costs more than a separate quantizer
// launch whose int8 result the workgroups copy (measured: 16.4 vs 11.6 us per call).
constexpr int kStreamQinPasses = 8;
// Producer waves of the streaming SwiGLU that also quantizes its output (32-row workgroups)
constexpr int kStreamQoutWaves = 8;
inline bool stream_qin_ok(int T, int K) {
  return K % kBlock == 0 && K / kBlock <= kStreamFoldWaveBlocks &&
         T * K <= kStreamQinPasses * 4 * stream_producers(K / kBlock);
}
constexpr int kGemmTileN = 128;  // weight rows per GEMM workgroup
constexpr int kGemmTileT = 128;  // tokens per GEMM workgroup
constexpr int kPadRows = 64;     // rows_pad is a multiple of this

enum WDType { WQ8 = 1, WQ4 = 2 };

// Device-resident weight in the repacked layout.
//   data:   [rows_pad/H][nb][H][G] bytes, G = 32 (q8: int8 row segment of one 32-block)
//                                       G = 16 (q4: the group's 16 bytes exactly as exported)
//   scales: q8 -> [rows_pad] f32 (per row)
//           q4 -> [rows_pad/H][nb][H] f32, the group scales as exported
// A (row n, block b) item sits at index ((n/H)*nb + b)*H + n%H, so a run of H rows of one
// block is contiguous and one H-row tile of all blocks is one contiguous chunk.
struct DevWeight {
  int dtype = 0;
  int H = 32;
  int64_t rows = 0, cols = 0, nb = 0, rows_pad = 0;
  uint8_t* data = nullptr;
  float* scales = nullptr;
  size_t data_bytes = 0, scale_bytes = 0;
};

__host__ __device__ inline int64_t item_index(int64_t n, int64_t b, int64_t nb, int H) {
  return ((n / H) * nb + b) * H + (n % H);
}

// ---------------------------------------------------------------- kernel argument blocks

struct GemvTarget {
  const uint8_t* data;
  const float* scales;
  float* y;          // [T][N]
  const float* res;  // [T][N] or null
  int N;
  int tiles;         // rows_pad / H
};

struct GemvArgs {
  GemvTarget tg[kMaxTargets];
  int tile_start[kMaxTargets + 1];  // prefix sums of tiles (matmul); swiglu uses tg[0]/tg[1]
  int n_targets;
  int total_tiles;
  int H;
  int tpw;            // tiles per workgroup (streaming kernel; tile_start then counts workgroups)
  int rsub;           // small kernel: rows per workgroup, a power of two dividing H (0: H); tile_start
                      // then counts workgroups
  const float* x;     // f32 [T][K] (quantized inside each workgroup) or null
  int stream;         // with x: the streaming kernel (else the small one) quantizes it
  const float* nw;    // small kernel: x is RMSNORM's input; nw [K] its weight, eps its epsilon
  float eps;
  const int8_t* xq;   // int8 [T][K] row-major (pre-quantized) when x is null
  const float* xd;    // f32 [T][nb]
  const int32_t* xs;  // int32 [T][nb] block sums of q
  int T, K, nb;
  // SwiGLU on the streaming kernel, one token, 32-row workgroups: the output row also quantized
  // (row-major int8 [N], block scales and block sums [N / 32], as the activation quantizer writes
  // them), or null
  int8_t* oq;
  float* od;
  int32_t* os;
};

struct GemmTarget {
  const uint8_t* data;
  const float* scales;
  float* y;
  const float* res;
  int N;
  int ntiles;  // ceil(rows_pad / kGemmTileN)
};

struct GemmArgs {
  GemmTarget tg[kMaxTargets];
  int tile_start[kMaxTargets + 1];
  int n_targets;
  int H;
  const int8_t* xq;  // MFMA B-fragment-major: [Tpad/32][nb][64 lanes][16 B]
  const float* xd;   // [nb][Tpad] (block mode) or [Tpad] (token mode)
  int T, Tpad, K, nb;
  int fast;          // 0: exact sequential mul+add; 1: fused multiply-add
  // SwiGLU (block mode): h also quantized into the next GEMM's operand, fragments [Tpad/32][onb][1 KB]
  // and block scales [onb][Tpad] (onb = N / 32), or null
  int8_t* oq;
  float* od;
  int onb;
};

struct F32Args {
  GemvTarget tg[kMaxTargets];
  int tile_start[kMaxTargets + 1];  // set by launch_f32act (in its kernel's row tiles)
  int n_targets;
  int H;
  const float* x;  // [T][K]
  int T, K, nb;
  const float* nw;  // T == 1, q4: x is RMSNORM's input, nw [K] its weight, eps its epsilon (else null)
  float eps;
  int rt;           // set by launch_f32act: rows per workgroup of the group-parallel q4 GEMV (divides H)
};

// ---------------------------------------------------------------- launchers (elmh_kernels.hip)

hipError_t launch_repack(const uint8_t* raw, const float* raw_scales, DevWeight& w, hipStream_t s);
// Row-major activation quantization: xq [T][K], xd [T][nb], xs [T][nb].
hipError_t launch_act_quant_rows(const float* x, int T, int K, int8_t* xq, float* xd, int32_t* xs, hipStream_t s);
// Fragment-major activation quantization for the MFMA GEMM: xq [Tpad/32][nb][1024], xd [nb][Tpad]
// (rows t >= T are written as zeros).
hipError_t launch_act_quant_frag(const float* x, int T, int Tpad, int K, int8_t* xq, float* xd, hipStream_t s);
hipError_t launch_rmsnorm_quant_frag(const float* x, const float* nw, float eps, int T, int Tpad, int K, int8_t* xq,
                                     float* xd, hipStream_t s);
// Per-token scale (extension): xq fragment-major as above, xd [Tpad].
hipError_t launch_act_quant_frag_token(const float* x, int T, int Tpad, int K, int8_t* xq, float* xd, hipStream_t s);

// Largest T the int8 GEMV path takes for this K (activation rows staged in LDS).
int gemv_max_tokens(int K);
// True if a workgroup may quantize T rows of K activations itself (small-matrix GEMV).
bool gemv_qin_ok(int T, int K);
// Items per thread of the streaming GEMV for a tile of `items` items (0: too many).
int gemv_stream_ipt(int dtype, int items, int producers);
size_t gemv_lds_bytes(int nt, int K, int nb, int H, int nsel);
bool gemm_qf_ok(int dtype, int T, int nb, int H, int N, int64_t rows_pad);
hipError_t launch_gemv_a8(int dtype, int swiglu, const GemvArgs& a, int total_tiles, hipStream_t s);
hipError_t launch_gemm_a8(int dtype, int swiglu, int token_mode, const GemmArgs& a, int total_tiles, hipStream_t s);
hipError_t launch_f32act(int dtype, int swiglu, const F32Args& a, hipStream_t s);
// True if launch_f32act runs the group-parallel q4 GEMV for this call (one token, q4 targets of tile
// height H, `rows` output rows, nsel = 2 for SwiGLU): its LDS, sized for the tile height the launch
// picks and, with norm (RMSNORM applied to x inside, a.nw), for the squares, fits a workgroup.
bool f32act_q4_ok(int T, int K, int nb, int H, int nsel, int rows, bool norm);
hipError_t launch_silu_mul(const float* g, const float* u, float* y, int64_t n, hipStream_t s);
// The non-matmul ops of a layer (elmh_layer.hip), same float order as edgelm's cpu backend.
hipError_t launch_rmsnorm(const float* x, const float* w, float* y, int rows, int dim, float eps, hipStream_t s);
// LDS a workgroup may allocate on gfx950 (160 KB per CU; kernels that use more than 64 KB raise their
// dynamic-LDS limit with hipFuncSetAttribute before the first launch)
constexpr size_t kMaxLds = 160 * 1024;
// dynamic LDS the attention kernels may take (their static LDS is a few words; this leaves 1 KB for it)
constexpr size_t kMaxAttnLds = kMaxLds - 1024;
size_t attention_lds_bytes(int hd, int n_max);
// Bytes of global score rows launch_attention needs for this call (0: the rows fit LDS). pos_dev: the
// position comes from device memory (rows sized for max_ctx).
size_t attention_global_score_bytes(int T, int pos0, bool pos_dev, int n_heads, int hd, int max_ctx);
// pos_dev (if not null): pos0 read from device memory (T must be 1; LDS sized for max_ctx).
// xq, xd, Tpad, quantized (all given): where the chunk kernel (T > 1, head size 64) runs, it also
// writes its output as the block-scale GEMM's activation fragments (xq, Tpad * n_heads * hd bytes)
// and scales (xd, 2 * n_heads * Tpad floats; tokens T .. Tpad-1 left as they were) and sets
// *quantized; otherwise *quantized is false and xq, xd are untouched.
// gscores: attention_global_score_bytes() of device memory where that is not 0 (score rows longer than
// LDS holds); without it such a call fails with hipErrorInvalidValue.
hipError_t launch_attention(const float* q, const float* k, const float* v, float* out, int T, int pos0,
                            const int* pos_dev, int n_heads, int n_kv, int hd, float* kc, float* vc, int max_ctx,
                            const float* rcos, const float* rsin, hipStream_t s, int8_t* xq = nullptr,
                            float* xd = nullptr, int Tpad = 0, bool* quantized = nullptr, float* gscores = nullptr);
hipError_t launch_embed(const int32_t* tok, int T, const DevWeight& w, float* y, hipStream_t s);
// dst[0, bytes) = value (a kernel: capturable in a HIP graph, unlike hipMemsetAsync)
hipError_t launch_fill(void* dst, int value, size_t bytes, hipStream_t s);
// measurement: every 16-byte word of src[0, bytes) read once (bytes and src 16-byte aligned), folded
// into sink (read_sweep_sink_bytes())
size_t read_sweep_sink_bytes();
hipError_t launch_read_sweep(const void* src, size_t bytes, void* sink, hipStream_t s);
hipError_t launch_argmax(const float* x, int rows, int64_t n, int32_t* out, hipStream_t s);
// one row's argmax over several workgroups (n <= 64 * 4096); with pos: ring[*pos & ring_mask] =
// the index, then *pos + 1. scratch: argmax_parts_scratch_bytes(), its last word zero before the
// first launch (each launch leaves it zero)
size_t argmax_parts_scratch_bytes();
hipError_t launch_argmax_parts(const float* x, int64_t n, int32_t* out, int32_t* pos, int32_t* ring, int ring_mask,
                               void* scratch, hipStream_t s);
// Measurement: `blocks` 256-thread workgroups of the rescale-ceiling kernel (mode 0 MFMA only, 1 q8 exact
// rescale, 2 q4 exact rescale), `iters` blocks per wave; sink: blocks * 256 floats.
hipError_t launch_rescale_ceiling(int mode, int blocks, int iters, float* sink, hipStream_t s);
// Test hook: S[t][n][b] for pre-quantized row-major activations.
hipError_t launch_block_sums(const DevWeight& w, const int8_t* xq, int T, int32_t* S, hipStream_t s);

}  // namespace elmh

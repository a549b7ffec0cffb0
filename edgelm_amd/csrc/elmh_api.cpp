// C-ABI layer of the delegate (include/elmh.h): contexts, weight upload + repack, scratch, and
// the dispatch of edgelm's matmul family onto the HIP kernels of elmh_kernels.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "elmh.h"
#include "elmh_internal.hpp"

using namespace elmh;

struct elmh_weight {
  DevWeight w;
};

namespace {

struct DevBuf {
  void* p = nullptr;
  size_t cap = 0;
};

thread_local std::string g_last_error;

// Scratch of elmh_matmul_noalloc_dev: a fixed device array, one copy per GPU the library runs on,
// held until the process ends. In host code `scratch` names a host-side stand-in, never a device
// address: elmh_create looks up each device's copy with hipGetSymbolAddress (that device current)
// and every host use goes through the pointer kept in g_noalloc_ptr.
constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
std::mutex g_noalloc_mu;
std::vector<unsigned char*> g_noalloc_ptr;  // per device id

}  // namespace

struct elmh_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string err;
  std::string arch;
  // staging for the host-pointer entry points
  DevBuf x, y, res;
  // activation-quantization scratch
  DevBuf xq, xd, xs;
  // SwiGLU fallback (gate/up of different layouts)
  DevBuf gu;
  // RMSNORM output when it cannot be fused into the matmul after it
  DevBuf nrm;
  // attention score rows longer than LDS holds
  DevBuf asc;
  // FFN pairs (elmh_ffn_dev): h quantized by the SwiGLU launch for the down projection
  DevBuf hq, hd, hs;
  // bumped whenever a scratch buffer above moves (a graph captured before then holds stale addresses)
  uint64_t scratch_gen = 0;
  // this device's copy of the no-allocation scratch array
  unsigned char* noalloc = nullptr;
  // whether the last elmh_attention_matmul_dev call had the attention kernel write the GEMM's operand
  int attn_fused = 0;
  // whether the last elmh_ffn_dev call had the SwiGLU launch quantize h for the down projection
  int ffn_fused = 0;
  // the one-row argmax's per-workgroup posts and counter (the counter zero between launches)
  void* argmax_scratch = nullptr;
};

namespace {

int fail(elmh_ctx* c, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  if (c) c->err = buf;
  return code;
}

#define HIP_OR_FAIL(ctx, call)                                                                              \
  do {                                                                                                      \
    hipError_t e_ = (call);                                                                                 \
    if (e_ != hipSuccess) return fail((ctx), ELMH_ERR_HIP, "%s: %s", #call, hipGetErrorString(e_));         \
  } while (0)

bool capturing(elmh_ctx* c) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(c->stream, &st) != hipSuccess) return false;
  return st != hipStreamCaptureStatusNone;
}

int ensure(elmh_ctx* c, DevBuf& b, size_t bytes) {
  if (bytes <= b.cap) return ELMH_OK;
  if (capturing(c)) return fail(c, ELMH_ERR_ARG, "scratch of %zu bytes needed during graph capture: call elmh_reserve first", bytes);
  if (b.p) {
    HIP_OR_FAIL(c, hipStreamSynchronize(c->stream));
    HIP_OR_FAIL(c, hipFree(b.p));
    b.p = nullptr;
    b.cap = 0;
  }
  const size_t cap = std::max<size_t>(bytes, 4096);
  ++c->scratch_gen;
  if (hipMalloc(&b.p, cap) != hipSuccess) return fail(c, ELMH_ERR_OOM, "hipMalloc(%zu) failed", cap);
  b.cap = cap;
  return ELMH_OK;
}

int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Rows per workgroup of the small GEMV (workgroup-quantizing, K <= 2048) for weights of H-row tiles:
// H (one tile per workgroup) unless ELMH_GEMV_ROWS names a power of two below it (same bits).
int small_rows(int H) {
  const char* v = getenv("ELMH_GEMV_ROWS");
  const int r = v && *v ? atoi(v) : 0;
  return r > 0 && r < H && !(r & (r - 1)) ? r : H;
}


// Row-tile height of the repacked layout, chosen from dtype and K only (so every weight sharing an
// input — MATMUL_N, gate/up — agrees). Short rows (K <= 2048) use 8-row tiles: many small decode
// workgroups with at most two items per thread. Rows of more than kStreamFoldWaveBlocks blocks
// also use 8-row tiles (the streaming GEMV's seven producer waves take a tile in eight batches).
// Other long rows use the tallest tile whose items fit the streaming GEMV's batches (q4: 2048
// items of 16 B, q8: 1024 items of 32 B), at least 4 rows.
int choose_H(int dtype, int64_t K) {
  const int64_t nb = (K + kBlock - 1) / kBlock;
  if (K <= 2048 || nb > kStreamFoldWaveBlocks) return 8;
  const int64_t cap = dtype == ELMH_Q4 ? 2048 : 1024;
  for (int H : {32, 16, 8})
    if (H * nb <= cap) return H;
  return 4;
}

// The repacked layout of a q8 / q4 weight (DevWeight): tile height, blocks, padded rows and bytes.
struct Layout {
  int H = 0;
  int64_t nb = 0, rows_pad = 0;
  size_t data_bytes = 0, scale_bytes = 0;
};
Layout layout_of(int dtype, int64_t rows, int64_t cols) {
  Layout L;
  L.nb = (cols + kBlock - 1) / kBlock;
  L.H = choose_H(dtype, cols);
  L.rows_pad = round_up(rows, kPadRows);
  L.data_bytes = (size_t)(L.rows_pad * L.nb * (dtype == ELMH_Q8 ? 32 : 16));
  L.scale_bytes = (size_t)(dtype == ELMH_Q8 ? L.rows_pad : L.rows_pad * L.nb) * sizeof(float);
  return L;
}
int check_weight(elmh_ctx* c, int dtype, int64_t rows, int64_t cols) {
  if (dtype != ELMH_Q8 && dtype != ELMH_Q4)
    return fail(c, ELMH_ERR_UNSUPPORTED, "dtype %d: only q8 (1) and q4 (2) weights are uploaded", dtype);
  if (rows < 1 || cols < 1) return fail(c, ELMH_ERR_ARG, "bad weight %lldx%lld", (long long)rows, (long long)cols);
  if (rows > (1ll << 30) || cols > (1ll << 24)) return fail(c, ELMH_ERR_UNSUPPORTED, "weight too large");
  if (dtype == ELMH_Q4 && cols % kBlock) return fail(c, ELMH_ERR_ARG, "q4 needs K %% 32 == 0, got K=%lld", (long long)cols);
  return ELMH_OK;
}

DevWeight new_weight(int dtype, int64_t rows, int64_t cols) {
  const Layout L = layout_of(dtype, rows, cols);
  DevWeight w;
  w.dtype = dtype;
  w.rows = rows;
  w.cols = cols;
  w.nb = L.nb;
  w.H = L.H;
  w.rows_pad = L.rows_pad;
  w.data_bytes = L.data_bytes;
  w.scale_bytes = L.scale_bytes;
  return w;
}

// Small-matrix decode path (workgroups quantize x themselves) vs the streaming path: short rows and
// at most ~4 MB of weights per launch.
bool use_small_gemv(int T, int64_t K, size_t bytes = 0) {
  return K <= 2048 && gemv_qin_ok(T, (int)K) && bytes <= (4u << 20);
}

bool a8_applies(const DevWeight& w) { return (w.dtype == ELMH_Q8 || w.dtype == ELMH_Q4) && w.cols % kBlock == 0; }

// Largest token count the int8 GEMV takes for this weight on the small (workgroup-quantized) or the
// streaming kernel, 0 if none.
int gemv_tokens(const DevWeight& w, int nsel, bool small) {
  const int K = (int)w.cols, nb = (int)w.nb;
  for (int nt : {4, 2, 1}) {
    if (nt > gemv_max_tokens(K)) continue;
    if (gemv_lds_bytes(nt, K, nb, w.H, nsel) > 64 * 1024) continue;
    if (small ? !use_small_gemv(nt, K)
              : gemv_stream_ipt(w.dtype, nsel * w.H * nb, stream_producers(nb)) == 0 || nt * w.H > kStreamFoldLanes)
      continue;
    return nt;
  }
  return 0;
}

int check_targets(elmh_ctx* c, int T, int64_t K, int n, elmh_weight* const* w, float* const* y) {
  if (T < 1 || K < 1) return fail(c, ELMH_ERR_ARG, "bad shape T=%d K=%lld", T, (long long)K);
  if (n < 1 || !w || !y) return fail(c, ELMH_ERR_ARG, "no targets");
  for (int i = 0; i < n; ++i) {
    if (!w[i] || !y[i]) return fail(c, ELMH_ERR_ARG, "target %d: null weight or output", i);
    if (w[i]->w.cols != K) return fail(c, ELMH_ERR_ARG, "target %d: K=%lld but weight has %lld columns", i, (long long)K, (long long)w[i]->w.cols);
  }
  return ELMH_OK;
}

// ---------------------------------------------------------------- device-pointer dispatch

// Tiles per workgroup of the streaming GEMV: enough items to fill the registers (q8 ~4, q4 ~8 per
// thread) while keeping at least two workgroups per CU.
int stream_tpw(const DevWeight& w, int T, int tiles_total, int nsel) {
  const int per_tile = nsel * w.H * (int)w.nb;
  const int target = kGemvThreads * (w.dtype == ELMH_Q8 ? 4 : 8);
  int tpw = std::max(1, target / per_tile);
  tpw = std::min(tpw, std::max(1, tiles_total / 512));
  while (tpw > 1 && (T * tpw * w.H > kStreamFoldLanes || gemv_stream_ipt(w.dtype, tpw * per_tile, stream_producers((int)w.nb)) == 0 ||
                     gemv_lds_bytes(T, (int)w.cols, (int)w.nb, tpw * w.H, nsel) > 64 * 1024))
    --tpw;
  return tpw;
}

// x (f32) goes to the small kernel, or with `stream` to the streaming one, which both quantize it
// per workgroup; otherwise xq / xd / xs hold the pre-quantized activation (streaming kernel).
int run_gemv_group(elmh_ctx* c, const float* x, const int8_t* xq, const float* xd, const int32_t* xs, int T,
                   int64_t K, const std::vector<int>& idx, elmh_weight* const* w, float* const* y,
                   const float* const* res, bool stream = false, const float* nw = nullptr, float eps = 0.f) {
  for (size_t i0 = 0; i0 < idx.size(); i0 += kMaxTargets) {
    GemvArgs a{};
    const size_t n = std::min<size_t>(kMaxTargets, idx.size() - i0);
    const DevWeight& w0 = w[idx[i0]]->w;
    int all_tiles = 0, tiles[kMaxTargets];
    for (size_t j = 0; j < n; ++j) all_tiles += tiles[j] = (int)(w[idx[i0 + j]]->w.rows_pad / w0.H);
    const bool small = x && !stream;
    a.tpw = small ? 1 : stream_tpw(w0, T, all_tiles, 1);
    a.rsub = small ? small_rows(w0.H) : 0;
    const int split = small ? w0.H / a.rsub : 1;  // small kernel: workgroups per tile
    int wgs = 0;
    a.H = w0.H;
    for (size_t j = 0; j < n; ++j) {
      const DevWeight& wd = w[idx[i0 + j]]->w;
      a.tg[j] = {wd.data, wd.scales, y[idx[i0 + j]], res ? res[idx[i0 + j]] : nullptr, (int)wd.rows, tiles[j]};
      a.tile_start[j] = wgs;
      wgs += small ? tiles[j] * split : (tiles[j] + a.tpw - 1) / a.tpw;
    }
    a.tile_start[n] = wgs;
    a.n_targets = (int)n;
    a.total_tiles = wgs;
    a.x = x;
    a.stream = stream;
    a.nw = nw;
    a.eps = eps;
    a.xq = xq;
    a.xd = xd;
    a.xs = xs;
    a.T = T;
    a.K = (int)K;
    a.nb = (int)(K / kBlock);
    HIP_OR_FAIL(c, launch_gemv_a8(w0.dtype, 0, a, wgs, c->stream));
  }
  return ELMH_OK;
}

int run_gemm_group(elmh_ctx* c, const int8_t* xq, const float* xd, int T, int Tpad, int64_t K,
                   const std::vector<int>& idx, elmh_weight* const* w, float* const* y, const float* const* res,
                   int token_mode, int fast) {
  for (size_t i0 = 0; i0 < idx.size(); i0 += kMaxTargets) {
    GemmArgs a{};
    const size_t n = std::min<size_t>(kMaxTargets, idx.size() - i0);
    int tiles = 0;
    const DevWeight& w0 = w[idx[i0]]->w;
    a.H = w0.H;
    for (size_t j = 0; j < n; ++j) {
      const DevWeight& wd = w[idx[i0 + j]]->w;
      a.tg[j] = {wd.data, wd.scales, y[idx[i0 + j]], res ? res[idx[i0 + j]] : nullptr, (int)wd.rows,
                 (int)((wd.rows_pad + kGemmTileN - 1) / kGemmTileN)};
      a.tile_start[j] = tiles;
      tiles += a.tg[j].ntiles;
    }
    a.tile_start[n] = tiles;
    a.n_targets = (int)n;
    a.xq = xq;
    a.xd = xd;
    a.T = T;
    a.Tpad = Tpad;
    a.K = (int)K;
    a.nb = (int)(K / kBlock);
    a.fast = fast;
    HIP_OR_FAIL(c, launch_gemm_a8(w0.dtype, 0, token_mode, a, tiles, c->stream));
  }
  return ELMH_OK;
}

int run_f32_group(elmh_ctx* c, const float* x, int T, int64_t K, const std::vector<int>& idx, elmh_weight* const* w,
                  float* const* y, const float* const* res, const float* nw = nullptr, float eps = 0.f) {
  for (size_t i0 = 0; i0 < idx.size(); i0 += kMaxTargets) {
    F32Args a{};
    const size_t n = std::min<size_t>(kMaxTargets, idx.size() - i0);
    int groups = 0;
    const DevWeight& w0 = w[idx[i0]]->w;
    a.H = w0.H;
    for (size_t j = 0; j < n; ++j) {
      const DevWeight& wd = w[idx[i0 + j]]->w;
      const int g = (int)((wd.rows + 255) / 256);
      a.tg[j] = {wd.data, wd.scales, y[idx[i0 + j]], res ? res[idx[i0 + j]] : nullptr, (int)wd.rows, g};
      a.tile_start[j] = groups;
      groups += g;
    }
    a.tile_start[n] = groups;
    a.n_targets = (int)n;
    a.x = x;
    a.T = T;
    a.K = (int)K;
    a.nb = (int)w0.nb;
    a.nw = nw;  // set only when f32_norm_fusable holds
    a.eps = eps;
    HIP_OR_FAIL(c, launch_f32act(w0.dtype, 0, a, c->stream));
  }
  return ELMH_OK;
}

// Where one call's quantized activation lives: the context's buffers (grown on demand), or with
// `fixed` set a region of fixed size carved into the same three parts (the no-allocation entry point).
struct Scratch {
  unsigned char* fixed = nullptr;
  size_t fixed_bytes = 0;
};
struct ActBufs {
  int8_t* q = nullptr;  // int8 values (row-major or GEMM fragments)
  float* d = nullptr;   // scales
  int32_t* s = nullptr; // block sums of q (row-major GEMV path only)
};

int act_buffers(elmh_ctx* c, const Scratch& sc, size_t q_bytes, size_t d_bytes, size_t s_bytes, ActBufs* out) {
  if (sc.fixed) {
    const size_t d_off = (size_t)round_up((int64_t)q_bytes, 256), s_off = (size_t)round_up((int64_t)(d_off + d_bytes), 256);
    const size_t need = s_off + s_bytes;
    if (need > sc.fixed_bytes)
      return fail(c, ELMH_ERR_ARG, "the activation needs %zu bytes of scratch; the no-allocation entry point has %zu",
                  need, sc.fixed_bytes);
    out->q = (int8_t*)sc.fixed;
    out->d = (float*)(sc.fixed + d_off);
    out->s = s_bytes ? (int32_t*)(sc.fixed + s_off) : nullptr;
    return ELMH_OK;
  }
  int rc;
  if ((rc = ensure(c, c->xq, q_bytes))) return rc;
  if ((rc = ensure(c, c->xd, d_bytes))) return rc;
  if (s_bytes && (rc = ensure(c, c->xs, s_bytes))) return rc;
  out->q = (int8_t*)c->xq.p;
  out->d = (float*)c->xd.p;
  out->s = s_bytes ? (int32_t*)c->xs.p : nullptr;
  return ELMH_OK;
}

// x quantized into the GEMM's fragments: every one of the Tpad token slots is written (zeros past T),
// so nothing left in the buffer by an earlier call is read
int quant_frag(elmh_ctx* c, const Scratch& sc, const float* x, int T, int64_t K, int token_mode, int* Tpad_out,
               ActBufs* a) {
  const int Tpad = (int)round_up(T, kGemmTileT);
  const int64_t nb = K / kBlock;
  int rc;
  if ((rc = act_buffers(c, sc, (size_t)Tpad * K, (size_t)Tpad * (token_mode ? 1 : nb) * sizeof(float), 0, a)))
    return rc;
  if (token_mode)
    HIP_OR_FAIL(c, launch_act_quant_frag_token(x, T, Tpad, (int)K, a->q, a->d, c->stream));
  else
    HIP_OR_FAIL(c, launch_act_quant_frag(x, T, Tpad, (int)K, a->q, a->d, c->stream));
  *Tpad_out = Tpad;
  return ELMH_OK;
}

// RMSNORM and the block-scale fragment quantization in one launch (K <= 2048)
int quant_frag_norm(elmh_ctx* c, const float* x, const float* nw, float eps, int T, int64_t K, int* Tpad_out,
                    ActBufs* a) {
  const int Tpad = (int)round_up(T, kGemmTileT);
  const int64_t nb = K / kBlock;
  int rc;
  if ((rc = act_buffers(c, Scratch{}, (size_t)Tpad * K, (size_t)Tpad * nb * sizeof(float), 0, a))) return rc;
  HIP_OR_FAIL(c, launch_rmsnorm_quant_frag(x, nw, eps, T, Tpad, (int)K, a->q, a->d, c->stream));
  *Tpad_out = Tpad;
  return ELMH_OK;
}

int quant_rows(elmh_ctx* c, const Scratch& sc, const float* x, int T, int64_t K, ActBufs* a) {
  const int64_t nb = K / kBlock;
  int rc;
  if ((rc = act_buffers(c, sc, (size_t)T * K, (size_t)T * nb * sizeof(float), (size_t)T * nb * sizeof(int32_t), a)))
    return rc;
  HIP_OR_FAIL(c, launch_act_quant_rows(x, T, (int)K, a->q, a->d, a->s, c->stream));
  return ELMH_OK;
}

// Groups target indices by dtype (one kernel instantiation per dtype).
std::vector<std::vector<int>> by_dtype(int n, elmh_weight* const* w) {
  std::vector<int> q8, q4;
  for (int i = 0; i < n; ++i) (w[i]->w.dtype == ELMH_Q8 ? q8 : q4).push_back(i);
  std::vector<std::vector<int>> g;
  if (!q8.empty()) g.push_back(q8);
  if (!q4.empty()) g.push_back(q4);
  return g;
}

int run_matmul(elmh_ctx* c, const float* x, int T, int64_t K, int n, elmh_weight* const* w, float* const* y,
               const float* const* res, int act, int mode, const Scratch& sc = Scratch{}) {
  int rc = check_targets(c, T, K, n, w, y);
  if (rc) return rc;
  if (act < ELMH_ACT_F32 || act > ELMH_ACT_INT8_TOKEN) return fail(c, ELMH_ERR_ARG, "bad act mode %d", act);
  bool a8 = act != ELMH_ACT_F32;
  for (int i = 0; i < n; ++i) a8 = a8 && a8_applies(w[i]->w);
  const auto groups = by_dtype(n, w);
  if (!a8) {
    for (const auto& g : groups)
      if ((rc = run_f32_group(c, x, T, K, g, w, y, res))) return rc;
    return ELMH_OK;
  }
  if (act == ELMH_ACT_INT8_TOKEN) {
    int Tpad;
    ActBufs ab;
    if ((rc = quant_frag(c, sc, x, T, K, 1, &Tpad, &ab))) return rc;
    for (const auto& g : groups)
      if ((rc = run_gemm_group(c, ab.q, ab.d, T, Tpad, K, g, w, y, res, 1, mode == ELMH_FAST)))
        return rc;
    return ELMH_OK;
  }
  size_t bytes = 0;
  for (int i = 0; i < n; ++i) bytes += w[i]->w.data_bytes + w[i]->w.scale_bytes;
  const bool qin = use_small_gemv(T, K, bytes);  // small rows: each workgroup quantizes x itself
  int nt = 4;
  for (int i = 0; i < n; ++i) nt = std::min(nt, gemv_tokens(w[i]->w, 1, qin));
  if (T <= nt) {
    // f32 x to the kernel (each workgroup quantizes it) unless it is too long for the streaming
    // kernel's registers: then one quantizer launch first
    const bool xin = qin || stream_qin_ok(T, (int)K);
    ActBufs ab;
    if (!xin && (rc = quant_rows(c, sc, x, T, K, &ab))) return rc;
    for (const auto& g : groups)
      if ((rc = run_gemv_group(c, xin ? x : nullptr, ab.q, ab.d, ab.s, T, K, g, w, y, res, !qin)))
        return rc;
    return ELMH_OK;
  }
  int Tpad;
  ActBufs ab;
  if ((rc = quant_frag(c, sc, x, T, K, 0, &Tpad, &ab))) return rc;
  for (const auto& g : groups)
    if ((rc = run_gemm_group(c, ab.q, ab.d, T, Tpad, K, g, w, y, res, 0, mode == ELMH_FAST)))
      return rc;
  return ELMH_OK;
}

// The SwiGLU output quantized for the next matmul by the SwiGLU launch itself: row-major as
// elmh_quantize_act_dev writes it (q, d, s; the one-token GEMV), or with `frag` as the block-scale
// GEMM's operand (fragments q [Tpad/32][N/32][1 KB], scales d [N/32][Tpad]); `done` is set when the
// SwiGLU launch wrote it.
struct QuantOut {
  int8_t* q;
  float* d;
  int32_t* s;
  bool frag;
  int Tpad;
  bool done;
};

// Whether the streaming SwiGLU can quantize its output in the fold (one token, 32-row workgroups of
// kStreamQoutWaves producer waves, x quantized per workgroup).
bool stream_qout_ok(const DevWeight& g, int K) {
  return g.H <= 32 && 32 % g.H == 0 && g.rows % 32 == 0 && g.nb <= kStreamFoldWaveBlocks && stream_qin_ok(1, K) &&
         gemv_stream_ipt(g.dtype, 2 * 32 * (int)g.nb, 64 * kStreamQoutWaves) != 0 &&
         gemv_lds_bytes(1, K, (int)g.nb, 32, 2) <= 64 * 1024;
}

int run_swiglu(elmh_ctx* c, const float* x, int T, int64_t K, const elmh_weight* wg, const elmh_weight* wu, float* y,
               int act, int mode, const float* nw = nullptr, float eps = 0.f, QuantOut* qo = nullptr) {
  if (!wg || !wu || !y) return fail(c, ELMH_ERR_ARG, "swiglu: null weight or output");
  if (T < 1 || wg->w.cols != K || wu->w.cols != K) return fail(c, ELMH_ERR_ARG, "swiglu: bad shape");
  if (wg->w.rows != wu->w.rows) return fail(c, ELMH_ERR_ARG, "swiglu: gate and up row counts differ");
  if (act < ELMH_ACT_F32 || act > ELMH_ACT_INT8_TOKEN) return fail(c, ELMH_ERR_ARG, "bad act mode %d", act);
  const DevWeight &g = wg->w, &u = wu->w;
  const bool a8 = act != ELMH_ACT_F32 && a8_applies(g) && a8_applies(u);
  int rc;
  if (g.dtype != u.dtype || g.H != u.H) {
    // different layouts: two matmuls into scratch, then the silu * up epilogue
    const size_t nel = (size_t)T * g.rows;
    if ((rc = ensure(c, c->gu, 2 * nel * sizeof(float)))) return rc;
    float* G = (float*)c->gu.p;
    float* Uo = G + nel;
    elmh_weight* ws[2] = {const_cast<elmh_weight*>(wg), const_cast<elmh_weight*>(wu)};
    float* ys[2] = {G, Uo};
    if ((rc = run_matmul(c, x, T, K, 2, ws, ys, nullptr, a8 ? act : ELMH_ACT_F32, mode))) return rc;
    HIP_OR_FAIL(c, launch_silu_mul(G, Uo, y, (int64_t)nel, c->stream));
    return ELMH_OK;
  }
  if (!a8) {
    F32Args a{};
    const int groups = (int)((g.rows + 255) / 256);
    a.tg[0] = {g.data, g.scales, y, nullptr, (int)g.rows, groups};
    a.tg[1] = {u.data, u.scales, y, nullptr, (int)u.rows, groups};
    a.tile_start[0] = 0;
    a.tile_start[1] = groups;
    a.n_targets = 1;
    a.H = g.H;
    a.x = x;
    a.T = T;
    a.K = (int)K;
    a.nb = (int)g.nb;
    a.nw = nw;  // set only when f32_norm_fusable holds
    a.eps = eps;
    HIP_OR_FAIL(c, launch_f32act(g.dtype, 1, a, c->stream));
    return ELMH_OK;
  }
  const bool qin = use_small_gemv(T, K, g.data_bytes + g.scale_bytes + u.data_bytes + u.scale_bytes);
  const int nt = gemv_tokens(g, 2, qin);
  if (nw && !(act == ELMH_ACT_INT8 && (T <= nt ? qin : K <= 2048)))
    return fail(c, ELMH_ERR_UNSUPPORTED, "swiglu: fused rmsnorm off the small GEMV and block-scale GEMM paths");
  if (act == ELMH_ACT_INT8 && T <= nt) {
    GemvArgs a{};
    const bool xin = qin || stream_qin_ok(T, (int)K);  // as in run_matmul
    ActBufs ab;
    if (!xin && (rc = quant_rows(c, Scratch{}, x, T, K, &ab))) return rc;
    const int tiles = (int)(g.rows_pad / g.H);
    // one token on the streaming kernel: 32-row workgroups of eight producer waves, which also
    // quantize the output row when the caller asks for it (8B gate+up alone: 15.5-15.9 -> 15.4 us)
    const bool w32 = !qin && xin && T == 1 && !nw && stream_qout_ok(g, (int)K);
    const bool qout = qo && !qo->frag && w32;
    a.tpw = w32 ? 32 / g.H : 1;
    a.rsub = qin ? small_rows(g.H) : 0;
    const int wgs = qin ? tiles * (g.H / a.rsub) : (tiles + a.tpw - 1) / a.tpw;
    a.tg[0] = {g.data, g.scales, y, nullptr, (int)g.rows, tiles};
    a.tg[1] = {u.data, u.scales, y, nullptr, (int)u.rows, tiles};
    a.n_targets = 2;
    a.total_tiles = wgs;
    a.H = g.H;
    if (qout) {
      a.oq = qo->q;
      a.od = qo->d;
      a.os = qo->s;
      qo->done = true;
    }
    a.x = xin ? x : nullptr;
    a.stream = !qin;
    a.nw = nw;  // set only when this small path applies (norm_fusable)
    a.eps = eps;
    a.xq = ab.q;
    a.xd = ab.d;
    a.xs = ab.s;
    a.T = T;
    a.K = (int)K;
    a.nb = (int)(K / kBlock);
    HIP_OR_FAIL(c, launch_gemv_a8(g.dtype, 1, a, wgs, c->stream));
    return ELMH_OK;
  }
  const int token = act == ELMH_ACT_INT8_TOKEN;
  int Tpad;
  ActBufs ab;
  if ((rc = nw ? quant_frag_norm(c, x, nw, eps, T, K, &Tpad, &ab) : quant_frag(c, Scratch{}, x, T, K, token, &Tpad, &ab)))
    return rc;
  GemmArgs a{};
  const int tiles = (int)((g.rows_pad + kGemmTileN - 1) / kGemmTileN);
  a.tg[0] = {g.data, g.scales, y, nullptr, (int)g.rows, tiles};
  a.tg[1] = {u.data, u.scales, y, nullptr, (int)u.rows, tiles};
  a.n_targets = 2;
  a.H = g.H;
  a.xq = ab.q;
  a.xd = ab.d;
  a.T = T;
  a.Tpad = Tpad;
  a.K = (int)K;
  a.nb = (int)(K / kBlock);
  a.fast = mode == ELMH_FAST;
  if (qo && qo->frag && !token && Tpad == qo->Tpad && gemm_qf_ok(g.dtype, T, a.nb, g.H, (int)g.rows, g.rows_pad)) {
    a.oq = qo->q;
    a.od = qo->d;
    a.onb = (int)(g.rows / kBlock);
    qo->done = true;
  }
  HIP_OR_FAIL(c, launch_gemm_a8(g.dtype, 1, token, a, tiles, c->stream));
  return ELMH_OK;
}

// True if RMSNORM of x can run inside the int8-activation small GEMV that consumes it: the small
// (workgroup-quantizing) kernel applies to every target at this T and K.
bool norm_fusable(int T, int64_t K, int n, const elmh_weight* const* w, int nsel, int act) {
  if (act != ELMH_ACT_INT8 || K % kBlock || K > 2048) return false;
  size_t bytes = 0;
  for (int i = 0; i < n; ++i) {
    if (!a8_applies(w[i]->w)) return false;
    bytes += w[i]->w.data_bytes + w[i]->w.scale_bytes;
  }
  if (!use_small_gemv(T, K, bytes)) return false;
  for (int i = 0; i < n; ++i)
    if (T > gemv_tokens(w[i]->w, nsel, true)) return false;
  return true;
}

// True if the int8-activation (block scales) call takes the GEMM at this T (more tokens than the
// GEMV takes) and K fits the fused RMSNORM + fragment quantizer.
// run_matmul / run_swiglu take the block-scale GEMM (fragments from act_quant_frag_kernel) for
// these targets: int8 block activations and too many tokens for the GEMV
bool block_gemm(int T, int64_t K, int n, const elmh_weight* const* w, int nsel, int act) {
  if (act != ELMH_ACT_INT8 || K % kBlock) return false;
  size_t bytes = 0;
  for (int i = 0; i < n; ++i) {
    if (!a8_applies(w[i]->w)) return false;
    bytes += w[i]->w.data_bytes + w[i]->w.scale_bytes;
  }
  const bool qin = use_small_gemv(T, K, bytes);
  int nt = 4;
  for (int i = 0; i < n; ++i) nt = std::min(nt, gemv_tokens(w[i]->w, nsel, qin));
  return T > nt;
}

// True if RMSNORM of x can run inside the f32-activation GEMV that consumes it (one token, q4
// targets of the group-parallel q4 GEMV's layout)
bool f32_norm_fusable(int T, int64_t K, int n, const elmh_weight* const* w, int nsel, int act) {
  if (act != ELMH_ACT_F32 || K > 8192) return false;
  int64_t rows = 0;  // launch_f32act's output rows: SwiGLU's gate rows, else every target's
  for (int i = 0; i < (nsel == 2 ? 1 : n); ++i) rows += w[i]->w.rows;
  for (int i = 0; i < n; ++i)
    if (w[i]->w.dtype != WQ4 || w[i]->w.H != w[0]->w.H ||
        !f32act_q4_ok(T, (int)K, (int)w[i]->w.nb, w[i]->w.H, nsel, (int)std::min<int64_t>(rows, 1 << 30), true))
      return false;
  return true;
}

bool norm_gemm(int T, int64_t K, int n, const elmh_weight* const* w, int nsel, int act) {
  return K <= 2048 && block_gemm(T, K, n, w, nsel, act);
}

// RMSNORM into the scratch buffer (the path when it cannot be fused)
int norm_to_scratch(elmh_ctx* c, const float* x, const float* nw, float eps, int T, int64_t K, const float** out) {
  int rc;
  if ((rc = ensure(c, c->nrm, (size_t)T * K * sizeof(float)))) return rc;
  HIP_OR_FAIL(c, launch_rmsnorm(x, nw, (float*)c->nrm.p, T, (int)K, eps, c->stream));
  *out = (const float*)c->nrm.p;
  return ELMH_OK;
}

struct DeviceGuard {
  explicit DeviceGuard(elmh_ctx* c) { (void)hipSetDevice(c->device); }
};

constexpr int kArgStepMaxN = 64 * 4096;  // launch_argmax_parts: 64 workgroups of 4096 values

int check_attention(elmh_ctx* c, const float* q, const float* k, const float* v, const float* out, int T, int pos0,
                    int n_heads, int n_kv, int head_dim, const float* k_cache, const float* v_cache, int max_ctx,
                    const float* rope_cos, const float* rope_sin) {
  if (!c || !q || !k || !v || !out || !k_cache || !v_cache) return fail(c, ELMH_ERR_ARG, "attention: null pointer");
  if (T < 1 || pos0 < 0 || (int64_t)pos0 + T > max_ctx)
    return fail(c, ELMH_ERR_ARG, "attention: context overflow (pos0 %d + T %d > max_ctx %d)", pos0, T, max_ctx);
  if (n_heads < 1 || n_kv < 1 || n_heads % n_kv || head_dim < 4 || head_dim % 4 || head_dim > 256)
    return fail(c, ELMH_ERR_ARG, "attention: heads %d / kv heads %d / head_dim %d", n_heads, n_kv, head_dim);
  if (!rope_cos != !rope_sin) return fail(c, ELMH_ERR_ARG, "attention: rope_cos and rope_sin go together");
  return ELMH_OK;
}

// The global score rows of an attention call whose rows do not fit LDS (null when they do).
int attention_scores(elmh_ctx* c, int T, int pos0, bool pos_dev, int n_heads, int head_dim, int max_ctx, float** out) {
  const size_t bytes = attention_global_score_bytes(T, pos0, pos_dev, n_heads, head_dim, max_ctx);
  *out = nullptr;
  if (!bytes) return ELMH_OK;
  if (const int rc = ensure(c, c->asc, bytes)) return rc;
  *out = static_cast<float*>(c->asc.p);
  return ELMH_OK;
}

}  // namespace

// ==================================================================== C ABI

extern "C" {

int elmh_device_count(int* count) {
  if (!count) return fail(nullptr, ELMH_ERR_ARG, "null count");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
  *count = n;
  return ELMH_OK;
}

int elmh_create(int device, elmh_ctx** out) {
  if (!out) return fail(nullptr, ELMH_ERR_ARG, "null out");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(nullptr, ELMH_ERR_NODEV, "no HIP device");
  if (device < 0 || device >= n) return fail(nullptr, ELMH_ERR_NODEV, "device %d out of range (%d devices)", device, n);
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return fail(nullptr, ELMH_ERR_NODEV, "hipGetDeviceProperties failed");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(nullptr, ELMH_ERR_NODEV, "device %d is %s; this library is built for gfx950 only", device, prop.gcnArchName);
  auto* c = new elmh_ctx();
  c->device = device;
  c->arch = prop.gcnArchName;
  if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return fail(nullptr, ELMH_ERR_HIP, "stream creation failed");
  }
  {
    // once per device, with the device current: the device address of its copy of `scratch`
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if ((size_t)device >= g_noalloc_ptr.size()) g_noalloc_ptr.resize((size_t)device + 1, nullptr);
    if (!g_noalloc_ptr[device]) {
      void* p = nullptr;
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        (void)hipStreamDestroy(c->stream);
        delete c;
        return fail(nullptr, ELMH_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
      }
      g_noalloc_ptr[device] = static_cast<unsigned char*>(p);
    }
    c->noalloc = g_noalloc_ptr[device];
  }
  if (hipMalloc(&c->argmax_scratch, argmax_parts_scratch_bytes()) != hipSuccess ||
      hipMemset(c->argmax_scratch, 0, argmax_parts_scratch_bytes()) != hipSuccess) {
    if (c->argmax_scratch) (void)hipFree(c->argmax_scratch);
    (void)hipStreamDestroy(c->stream);
    delete c;
    return fail(nullptr, ELMH_ERR_HIP, "argmax scratch allocation failed on device %d", device);
  }
  *out = c;
  return ELMH_OK;
}

void elmh_destroy(elmh_ctx* c) {
  if (!c) return;
  DeviceGuard g(c);
  (void)hipStreamSynchronize(c->stream);
  for (DevBuf* b : {&c->x, &c->y, &c->res, &c->xq, &c->xd, &c->xs, &c->gu, &c->nrm, &c->asc, &c->hq, &c->hd, &c->hs})
    if (b->p) (void)hipFree(b->p);
  if (c->argmax_scratch) (void)hipFree(c->argmax_scratch);
  (void)hipStreamDestroy(c->stream);
  delete c;
}

const char* elmh_last_error(const elmh_ctx* c) { return c ? c->err.c_str() : g_last_error.c_str(); }

const char* elmh_device_arch(const elmh_ctx* c) { return c ? c->arch.c_str() : ""; }

int elmh_upload_weight(elmh_ctx* c, int dtype, int64_t rows, int64_t cols, const void* data, const float* scales,
                       elmh_weight** out) {
  if (!c || !out) return fail(c, ELMH_ERR_ARG, "null ctx/out");
  *out = nullptr;
  int rc = check_weight(c, dtype, rows, cols);
  if (rc) return rc;
  if (!data || !scales) return fail(c, ELMH_ERR_ARG, "null weight data/scales");
  DeviceGuard guard(c);
  DevWeight w = new_weight(dtype, rows, cols);
  const size_t raw_bytes = (size_t)(dtype == ELMH_Q8 ? rows * cols : rows * (cols / 2));
  const size_t raw_sbytes = (size_t)(dtype == ELMH_Q8 ? rows : rows * w.nb) * sizeof(float);
  void *raw = nullptr, *raw_s = nullptr;
  auto cleanup = [&]() {
    if (raw) (void)hipFree(raw);
    if (raw_s) (void)hipFree(raw_s);
    if (w.data) (void)hipFree(w.data);
    if (w.scales) (void)hipFree(w.scales);
  };
  if (hipMalloc((void**)&w.data, w.data_bytes) != hipSuccess || hipMalloc((void**)&w.scales, w.scale_bytes) != hipSuccess ||
      hipMalloc(&raw, raw_bytes) != hipSuccess || hipMalloc(&raw_s, raw_sbytes) != hipSuccess) {
    cleanup();
    return fail(c, ELMH_ERR_OOM, "hipMalloc failed for a %lldx%lld weight", (long long)rows, (long long)cols);
  }
  hipError_t e = hipMemcpyAsync(raw, data, raw_bytes, hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(raw_s, scales, raw_sbytes, hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess) e = launch_repack((const uint8_t*)raw, (const float*)raw_s, w, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  (void)hipFree(raw);
  (void)hipFree(raw_s);
  raw = raw_s = nullptr;
  if (e != hipSuccess) {
    cleanup();
    return fail(c, ELMH_ERR_HIP, "weight upload: %s", hipGetErrorString(e));
  }
  *out = new elmh_weight{w};
  return ELMH_OK;
}

int elmh_free_weight(elmh_ctx* c, elmh_weight* w) {
  if (!w) return ELMH_OK;
  if (c) {
    DeviceGuard g(c);
    (void)hipStreamSynchronize(c->stream);
  }
  if (w->w.data) (void)hipFree(w->w.data);
  if (w->w.scales) (void)hipFree(w->w.scales);
  delete w;
  return ELMH_OK;
}

size_t elmh_weight_bytes(const elmh_weight* w) { return w ? w->w.data_bytes + w->w.scale_bytes : 0; }

int elmh_weight_layout(int dtype, int64_t rows, int64_t cols, int* H, size_t* data_bytes, size_t* scale_bytes) {
  int rc = check_weight(nullptr, dtype, rows, cols);
  if (rc) return rc;
  const Layout L = layout_of(dtype, rows, cols);
  if (H) *H = L.H;
  if (data_bytes) *data_bytes = L.data_bytes;
  if (scale_bytes) *scale_bytes = L.scale_bytes;
  return ELMH_OK;
}

// repack_kernel's permutation on the host: item (row n, block b) at item_index(n, b, nb, H), q8 rows
// zero-padded past K and past the last row, q4 padding rows 0x88 (q = 0) with scale 0.
int elmh_repack_host(int dtype, int64_t rows, int64_t cols, const void* data, const float* scales, void* out_data,
                     float* out_scales) {
  int rc = check_weight(nullptr, dtype, rows, cols);
  if (rc) return rc;
  if (!data || !scales || !out_data || !out_scales) return fail(nullptr, ELMH_ERR_ARG, "repack: null pointer");
  const Layout L = layout_of(dtype, rows, cols);
  const uint8_t* raw = static_cast<const uint8_t*>(data);
  uint8_t* out = static_cast<uint8_t*>(out_data);
  const int G = dtype == ELMH_Q8 ? 32 : 16;
  for (int64_t n = 0; n < L.rows_pad; ++n) {
    const bool real = n < rows;
    if (dtype == ELMH_Q8) out_scales[n] = real ? scales[n] : 0.f;
    for (int64_t b = 0; b < L.nb; ++b) {
      const int64_t dst = item_index(n, b, L.nb, L.H);
      uint8_t* o = out + dst * G;
      if (dtype == ELMH_Q8) {
        const int64_t k0 = b * kBlock, nk = real ? std::min<int64_t>(kBlock, cols - k0) : 0;
        if (nk > 0) std::memcpy(o, raw + n * cols + k0, (size_t)nk);
        std::memset(o + std::max<int64_t>(nk, 0), 0, (size_t)(kBlock - std::max<int64_t>(nk, 0)));
      } else {
        if (real)
          std::memcpy(o, raw + n * (cols / 2) + b * 16, 16);
        else
          std::memset(o, 0x88, 16);
        out_scales[dst] = real ? scales[n * L.nb + b] : 0.f;
      }
    }
  }
  return ELMH_OK;
}

int elmh_upload_weight_image(elmh_ctx* c, int dtype, int64_t rows, int64_t cols, const void* data, const float* scales,
                             elmh_weight** out) {
  if (!c || !out) return fail(c, ELMH_ERR_ARG, "null ctx/out");
  *out = nullptr;
  int rc = check_weight(c, dtype, rows, cols);
  if (rc) return rc;
  if (!data || !scales) return fail(c, ELMH_ERR_ARG, "null weight image");
  DeviceGuard guard(c);
  DevWeight w = new_weight(dtype, rows, cols);
  if (hipMalloc((void**)&w.data, w.data_bytes) != hipSuccess || hipMalloc((void**)&w.scales, w.scale_bytes) != hipSuccess) {
    if (w.data) (void)hipFree(w.data);
    if (w.scales) (void)hipFree(w.scales);
    return fail(c, ELMH_ERR_OOM, "hipMalloc failed for a %lldx%lld weight", (long long)rows, (long long)cols);
  }
  hipError_t e = hipMemcpyAsync(w.data, data, w.data_bytes, hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(w.scales, scales, w.scale_bytes, hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) {
    (void)hipFree(w.data);
    (void)hipFree(w.scales);
    return fail(c, ELMH_ERR_HIP, "weight image upload: %s", hipGetErrorString(e));
  }
  *out = new elmh_weight{w};
  return ELMH_OK;
}

int elmh_download_weight_image(elmh_ctx* c, const elmh_weight* w, void* data, float* scales) {
  if (!c || !w || !data || !scales) return fail(c, ELMH_ERR_ARG, "null ctx/weight/output");
  DeviceGuard guard(c);
  HIP_OR_FAIL(c, hipMemcpyAsync(data, w->w.data, w->w.data_bytes, hipMemcpyDeviceToHost, c->stream));
  HIP_OR_FAIL(c, hipMemcpyAsync(scales, w->w.scales, w->w.scale_bytes, hipMemcpyDeviceToHost, c->stream));
  HIP_OR_FAIL(c, hipStreamSynchronize(c->stream));
  return ELMH_OK;
}

uint64_t elmh_scratch_generation(const elmh_ctx* c) { return c ? c->scratch_gen : 0; }

int elmh_reserve(elmh_ctx* c, int max_T, int64_t max_K) {
  if (!c || max_T < 1 || max_K < 1) return fail(c, ELMH_ERR_ARG, "bad reserve");
  DeviceGuard g(c);
  const int64_t Tpad = round_up(max_T, kGemmTileT);
  const int64_t nb = (max_K + kBlock - 1) / kBlock;
  int rc;
  if ((rc = ensure(c, c->xq, (size_t)(Tpad * max_K)))) return rc;
  if ((rc = ensure(c, c->xd, (size_t)(Tpad * nb) * sizeof(float)))) return rc;
  if ((rc = ensure(c, c->xs, (size_t)(Tpad * nb) * sizeof(int32_t)))) return rc;
  if (max_K <= 8192 && (rc = ensure(c, c->nrm, (size_t)max_T * max_K * sizeof(float)))) return rc;
  return ELMH_OK;
}

int elmh_matmul_dev(elmh_ctx* c, const float* x, int T, int64_t K, int n, elmh_weight* const* w, float* const* y,
                    const float* const* res, int act, int mode) {
  if (!c || !x) return fail(c, ELMH_ERR_ARG, "null ctx/x");
  DeviceGuard g(c);
  return run_matmul(c, x, T, K, n, w, y, res, act, mode);
}

int elmh_matmul_noalloc_dev(elmh_ctx* c, const float* x, int T, int64_t K, int n, elmh_weight* const* w,
                            float* const* y, const float* const* res, int act, int mode) {
  if (!c || !x) return fail(c, ELMH_ERR_ARG, "null ctx/x");
  if (!c->noalloc) return fail(c, ELMH_ERR_HIP, "no-allocation scratch missing on device %d", c->device);
  DeviceGuard g(c);
  return run_matmul(c, x, T, K, n, w, y, res, act, mode, Scratch{c->noalloc, kNoAllocScratchBytes});
}

int elmh_swiglu_dev(elmh_ctx* c, const float* x, int T, int64_t K, const elmh_weight* wg, const elmh_weight* wu,
                    float* y, int act, int mode) {
  if (!c || !x) return fail(c, ELMH_ERR_ARG, "null ctx/x");
  DeviceGuard g(c);
  return run_swiglu(c, x, T, K, wg, wu, y, act, mode);
}

int elmh_swiglu_quant_dev(elmh_ctx* c, const float* x, int T, int64_t K, const elmh_weight* wg, const elmh_weight* wu,
                          float* y, int8_t* q, float* d, int32_t* s) {
  if (!c || !x || !q || !d || !s) return fail(c, ELMH_ERR_ARG, "null argument");
  if (!wg || wg->w.rows % kBlock) return fail(c, ELMH_ERR_ARG, "swiglu_quant: output rows must be a multiple of 32");
  DeviceGuard g(c);
  QuantOut qo{q, d, s, false, 0, false};
  int rc = run_swiglu(c, x, T, K, wg, wu, y, ELMH_ACT_INT8, ELMH_EXACT, nullptr, 0.f, &qo);
  if (rc) return rc;
  if (!qo.done) HIP_OR_FAIL(c, launch_act_quant_rows(y, T, (int)wg->w.rows, q, d, s, c->stream));
  return ELMH_OK;
}

int elmh_rmsnorm_matmul_dev(elmh_ctx* c, const float* x, const float* norm_w, float eps, int T, int64_t K, int n,
                            elmh_weight* const* w, float* const* y, const float* const* res, int act, int mode) {
  if (!c || !x || !norm_w) return fail(c, ELMH_ERR_ARG, "null ctx/x/norm weight");
  int rc = check_targets(c, T, K, n, w, y);
  if (rc) return rc;
  if (K > 8192) return fail(c, ELMH_ERR_ARG, "rmsnorm: dim %lld (1 .. 8192)", (long long)K);
  DeviceGuard g(c);
  if (norm_fusable(T, K, n, w, 1, act)) {
    for (const auto& grp : by_dtype(n, w))
      if ((rc = run_gemv_group(c, x, nullptr, nullptr, nullptr, T, K, grp, w, y, res, false, norm_w, eps))) return rc;
    return ELMH_OK;
  }
  if (f32_norm_fusable(T, K, n, w, 1, act)) {
    for (const auto& grp : by_dtype(n, w))
      if ((rc = run_f32_group(c, x, T, K, grp, w, y, res, norm_w, eps))) return rc;
    return ELMH_OK;
  }
  if (norm_gemm(T, K, n, w, 1, act)) {  // the block-scale GEMM: RMSNORM inside its quantizer launch
    int Tpad;
    ActBufs ab;
    if ((rc = quant_frag_norm(c, x, norm_w, eps, T, K, &Tpad, &ab))) return rc;
    for (const auto& grp : by_dtype(n, w))
      if ((rc = run_gemm_group(c, ab.q, ab.d, T, Tpad, K, grp, w, y, res, 0, mode == ELMH_FAST)))
        return rc;
    return ELMH_OK;
  }
  const float* xn;
  if ((rc = norm_to_scratch(c, x, norm_w, eps, T, K, &xn))) return rc;
  return run_matmul(c, xn, T, K, n, w, y, res, act, mode);
}

// RMSNORM then FFN_SWIGLU: RMSNORM inside the SwiGLU's launch where that kernel path normalizes rows
// itself, else into scratch first
int run_rmsnorm_swiglu(elmh_ctx* c, const float* x, const float* norm_w, float eps, int T, int64_t K,
                       const elmh_weight* wg, const elmh_weight* wu, float* y, int act, int mode, QuantOut* qo = nullptr) {
  const elmh_weight* const ws[2] = {wg, wu};
  if (wg->w.dtype == wu->w.dtype && wg->w.H == wu->w.H && wg->w.rows == wu->w.rows && wg->w.cols == K &&
      wu->w.cols == K &&
      (norm_fusable(T, K, 2, ws, 2, act) || norm_gemm(T, K, 2, ws, 2, act) || f32_norm_fusable(T, K, 2, ws, 2, act)))
    return run_swiglu(c, x, T, K, wg, wu, y, act, mode, norm_w, eps, qo);
  const float* xn;
  int rc;
  if ((rc = norm_to_scratch(c, x, norm_w, eps, T, K, &xn))) return rc;
  return run_swiglu(c, xn, T, K, wg, wu, y, act, mode, nullptr, 0.f, qo);
}

int elmh_rmsnorm_swiglu_dev(elmh_ctx* c, const float* x, const float* norm_w, float eps, int T, int64_t K,
                            const elmh_weight* wg, const elmh_weight* wu, float* y, int act, int mode) {
  if (!c || !x || !norm_w || !wg || !wu || !y) return fail(c, ELMH_ERR_ARG, "null ctx/x/norm weight/weight/y");
  if (T < 1 || K < 1 || K > 8192) return fail(c, ELMH_ERR_ARG, "rmsnorm: bad shape T=%d dim=%lld", T, (long long)K);
  DeviceGuard g(c);
  return run_rmsnorm_swiglu(c, x, norm_w, eps, T, K, wg, wu, y, act, mode);
}

int elmh_ffn_dev(elmh_ctx* c, const float* x, const float* norm_w, float eps, int T, int64_t K, const elmh_weight* wg,
                 const elmh_weight* wu, float* h, elmh_weight* wd, float* y, const float* res, int act, int mode) {
  if (!c || !x || !wg || !wu || !h || !wd || !y) return fail(c, ELMH_ERR_ARG, "null ctx/x/weight/h/y");
  if (norm_w && (T < 1 || K < 1 || K > 8192))
    return fail(c, ELMH_ERR_ARG, "rmsnorm: bad shape T=%d dim=%lld", T, (long long)K);
  const int64_t N = wg->w.rows;
  elmh_weight* const ws[1] = {wd};
  float* const ys[1] = {y};
  const float* const rs[1] = {res};
  int rc = check_targets(c, T, N, 1, ws, ys);
  if (rc) return rc;
  if (act < ELMH_ACT_F32 || act > ELMH_ACT_INT8_TOKEN) return fail(c, ELMH_ERR_ARG, "bad act mode %d", act);
  DeviceGuard g(c);
  c->ffn_fused = 0;
  // h quantized by the SwiGLU launch where the down projection then takes it pre-quantized: at one
  // token the streaming SwiGLU writes it row-major for the GEMV; on the block-scale GEMM path the
  // SwiGLU GEMM writes the down GEMM's fragments
  const size_t onb = (size_t)(N / kBlock);
  const bool down_a8 = act == ELMH_ACT_INT8 && N % kBlock == 0 && a8_applies(wd->w);
  const bool down_gemm =
      down_a8 && T > gemv_tokens(wd->w, 1, use_small_gemv(T, N, wd->w.data_bytes + wd->w.scale_bytes));
  const int Tpad = (int)round_up(T, kGemmTileT);
  QuantOut qo{nullptr, nullptr, nullptr, false, 0, false};
  bool try_q = false;
  if (down_a8 && T == 1 && gemv_tokens(wd->w, 1, false) >= T) {
    if ((rc = ensure(c, c->hq, (size_t)T * N)) || (rc = ensure(c, c->hd, (size_t)T * onb * sizeof(float))) ||
        (rc = ensure(c, c->hs, (size_t)T * onb * sizeof(int32_t))))
      return rc;
    qo = {(int8_t*)c->hq.p, (float*)c->hd.p, (int32_t*)c->hs.p, false, 0, false};
    try_q = true;
  } else if (down_gemm) {
    if ((rc = ensure(c, c->hq, (size_t)Tpad * N)) || (rc = ensure(c, c->hd, onb * Tpad * sizeof(float)))) return rc;
    qo = {(int8_t*)c->hq.p, (float*)c->hd.p, nullptr, true, Tpad, false};
    try_q = true;
  }
  rc = norm_w ? run_rmsnorm_swiglu(c, x, norm_w, eps, T, K, wg, wu, h, act, mode, try_q ? &qo : nullptr)
              : run_swiglu(c, x, T, K, wg, wu, h, act, mode, nullptr, 0.f, try_q ? &qo : nullptr);
  if (rc) return rc;
  if (!qo.done) return run_matmul(c, h, T, N, 1, ws, ys, res ? rs : nullptr, act, mode);
  c->ffn_fused = 1;
  const std::vector<int> idx = {0};
  if (qo.frag) return run_gemm_group(c, qo.q, qo.d, T, Tpad, N, idx, ws, ys, res ? rs : nullptr, 0, mode == ELMH_FAST);
  return run_gemv_group(c, nullptr, qo.q, qo.d, qo.s, T, N, idx, ws, ys, res ? rs : nullptr);
}

int elmh_ffn_fused(const elmh_ctx* c) { return c ? c->ffn_fused : 0; }

int elmh_matmul(elmh_ctx* c, const float* x, int T, int64_t K, int n, elmh_weight* const* w, float* const* y,
                const float* const* res, int act, int mode) {
  if (!c || !x) return fail(c, ELMH_ERR_ARG, "null ctx/x");
  int rc = check_targets(c, T, K, n, w, y);
  if (rc) return rc;
  DeviceGuard g(c);
  size_t ytot = 0;
  for (int i = 0; i < n; ++i) ytot += (size_t)T * w[i]->w.rows;
  if ((rc = ensure(c, c->x, (size_t)T * K * sizeof(float)))) return rc;
  if ((rc = ensure(c, c->y, ytot * sizeof(float)))) return rc;
  bool any_res = false;
  for (int i = 0; res && i < n; ++i) any_res = any_res || res[i];
  if (any_res && (rc = ensure(c, c->res, ytot * sizeof(float)))) return rc;
  HIP_OR_FAIL(c, hipMemcpyAsync(c->x.p, x, (size_t)T * K * sizeof(float), hipMemcpyHostToDevice, c->stream));
  std::vector<float*> dy(n);
  std::vector<const float*> dr(n, nullptr);
  size_t off = 0;
  for (int i = 0; i < n; ++i) {
    const size_t cnt = (size_t)T * w[i]->w.rows;
    dy[i] = (float*)c->y.p + off;
    if (any_res && res[i]) {
      dr[i] = (float*)c->res.p + off;
      HIP_OR_FAIL(c, hipMemcpyAsync((void*)dr[i], res[i], cnt * sizeof(float), hipMemcpyHostToDevice, c->stream));
    }
    off += cnt;
  }
  if ((rc = run_matmul(c, (const float*)c->x.p, T, K, n, w, dy.data(), any_res ? dr.data() : nullptr, act, mode)))
    return rc;
  for (int i = 0; i < n; ++i)
    HIP_OR_FAIL(c, hipMemcpyAsync(y[i], dy[i], (size_t)T * w[i]->w.rows * sizeof(float), hipMemcpyDeviceToHost, c->stream));
  HIP_OR_FAIL(c, hipStreamSynchronize(c->stream));
  return ELMH_OK;
}

int elmh_swiglu(elmh_ctx* c, const float* x, int T, int64_t K, const elmh_weight* wg, const elmh_weight* wu, float* y,
                int act, int mode) {
  if (!c || !x || !wg || !wu || !y) return fail(c, ELMH_ERR_ARG, "null argument");
  if (T < 1) return fail(c, ELMH_ERR_ARG, "bad T");
  DeviceGuard g(c);
  int rc;
  const size_t ny = (size_t)T * wg->w.rows;
  if ((rc = ensure(c, c->x, (size_t)T * K * sizeof(float)))) return rc;
  if ((rc = ensure(c, c->y, ny * sizeof(float)))) return rc;
  HIP_OR_FAIL(c, hipMemcpyAsync(c->x.p, x, (size_t)T * K * sizeof(float), hipMemcpyHostToDevice, c->stream));
  if ((rc = run_swiglu(c, (const float*)c->x.p, T, K, wg, wu, (float*)c->y.p, act, mode))) return rc;
  HIP_OR_FAIL(c, hipMemcpyAsync(y, c->y.p, ny * sizeof(float), hipMemcpyDeviceToHost, c->stream));
  HIP_OR_FAIL(c, hipStreamSynchronize(c->stream));
  return ELMH_OK;
}

int elmh_quantize_act_dev(elmh_ctx* c, const float* x, int T, int64_t K, int8_t* q, float* d, int32_t* s) {
  if (!c || !x || !q || !d || !s || T < 1 || K < kBlock || K % kBlock) return fail(c, ELMH_ERR_ARG, "bad quantize_act args");
  DeviceGuard g(c);
  HIP_OR_FAIL(c, launch_act_quant_rows(x, T, (int)K, q, d, s, c->stream));
  return ELMH_OK;
}

int elmh_gemv_a8_dev(elmh_ctx* c, const int8_t* q, const float* d, const int32_t* s, int T, int64_t K, int n,
                     elmh_weight* const* w, float* const* y, const float* const* res) {
  if (!c || !q || !d || !s) return fail(c, ELMH_ERR_ARG, "null argument");
  int rc = check_targets(c, T, K, n, w, y);
  if (rc) return rc;
  for (int i = 0; i < n; ++i)
    if (!a8_applies(w[i]->w)) return fail(c, ELMH_ERR_ARG, "target %d: int8 GEMV needs K %% 32 == 0", i);
  int nt = 4;
  for (int i = 0; i < n; ++i) nt = std::min(nt, gemv_tokens(w[i]->w, 1, false));
  if (T > nt) return fail(c, ELMH_ERR_UNSUPPORTED, "int8 GEMV takes at most %d tokens at K=%lld", nt, (long long)K);
  DeviceGuard g(c);
  for (const auto& grp : by_dtype(n, w))
    if ((rc = run_gemv_group(c, nullptr, q, d, s, T, K, grp, w, y, res))) return rc;
  return ELMH_OK;
}

int elmh_quantize_act(elmh_ctx* c, const float* x, int T, int64_t K, int8_t* q, float* d) {
  if (!c || !x || !q || !d || T < 1 || K < kBlock || K % kBlock) return fail(c, ELMH_ERR_ARG, "bad quantize_act args");
  DeviceGuard g(c);
  int rc;
  const int64_t nb = K / kBlock;
  if ((rc = ensure(c, c->x, (size_t)T * K * sizeof(float)))) return rc;
  HIP_OR_FAIL(c, hipMemcpyAsync(c->x.p, x, (size_t)T * K * sizeof(float), hipMemcpyHostToDevice, c->stream));
  ActBufs ab;
  if ((rc = quant_rows(c, Scratch{}, (const float*)c->x.p, T, K, &ab))) return rc;
  HIP_OR_FAIL(c, hipMemcpyAsync(q, ab.q, (size_t)T * K, hipMemcpyDeviceToHost, c->stream));
  HIP_OR_FAIL(c, hipMemcpyAsync(d, ab.d, (size_t)T * nb * sizeof(float), hipMemcpyDeviceToHost, c->stream));
  HIP_OR_FAIL(c, hipStreamSynchronize(c->stream));
  return ELMH_OK;
}

int elmh_block_sums(elmh_ctx* c, const int8_t* xq, int T, const elmh_weight* w, int32_t* S) {
  if (!c || !xq || !w || !S || T < 1) return fail(c, ELMH_ERR_ARG, "null argument");
  if (!a8_applies(w->w)) return fail(c, ELMH_ERR_ARG, "block sums need K %% 32 == 0");
  DeviceGuard g(c);
  int rc;
  const size_t nS = (size_t)T * w->w.rows * w->w.nb;
  if ((rc = ensure(c, c->xq, (size_t)T * w->w.cols))) return rc;
  if ((rc = ensure(c, c->y, nS * sizeof(int32_t)))) return rc;
  HIP_OR_FAIL(c, hipMemcpyAsync(c->xq.p, xq, (size_t)T * w->w.cols, hipMemcpyHostToDevice, c->stream));
  HIP_OR_FAIL(c, launch_block_sums(w->w, (const int8_t*)c->xq.p, T, (int32_t*)c->y.p, c->stream));
  HIP_OR_FAIL(c, hipMemcpyAsync(S, c->y.p, nS * sizeof(int32_t), hipMemcpyDeviceToHost, c->stream));
  HIP_OR_FAIL(c, hipStreamSynchronize(c->stream));
  return ELMH_OK;
}

// ---- plumbing ----

int elmh_malloc(elmh_ctx* c, size_t bytes, void** p) {
  if (!c || !p) return fail(c, ELMH_ERR_ARG, "null argument");
  DeviceGuard g(c);
  if (hipMalloc(p, bytes ? bytes : 1) != hipSuccess) return fail(c, ELMH_ERR_OOM, "hipMalloc(%zu) failed", bytes);
  return ELMH_OK;
}

int elmh_free(elmh_ctx* c, void* p) {
  if (!c) return fail(c, ELMH_ERR_ARG, "null ctx");
  DeviceGuard g(c);
  HIP_OR_FAIL(c, hipStreamSynchronize(c->stream));
  if (p) HIP_OR_FAIL(c, hipFree(p));
  return ELMH_OK;
}

int elmh_memcpy_h2d(elmh_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c) return fail(c, ELMH_ERR_ARG, "null ctx");
  DeviceGuard g(c);
  HIP_OR_FAIL(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
  HIP_OR_FAIL(c, hipStreamSynchronize(c->stream));
  return ELMH_OK;
}

int elmh_memcpy_d2h(elmh_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c) return fail(c, ELMH_ERR_ARG, "null ctx");
  DeviceGuard g(c);
  HIP_OR_FAIL(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
  HIP_OR_FAIL(c, hipStreamSynchronize(c->stream));
  return ELMH_OK;
}

int elmh_host_alloc(elmh_ctx* c, size_t bytes, void** ptr) {
  if (!c || !ptr) return fail(c, ELMH_ERR_ARG, "null ctx/ptr");
  *ptr = nullptr;
  DeviceGuard g(c);
  if (hipHostMalloc(ptr, std::max<size_t>(bytes, 64), hipHostMallocDefault) != hipSuccess)
    return fail(c, ELMH_ERR_OOM, "hipHostMalloc(%zu) failed", bytes);
  return ELMH_OK;
}

int elmh_host_free(elmh_ctx* c, void* ptr) {
  if (!c) return fail(c, ELMH_ERR_ARG, "null ctx");
  if (!ptr) return ELMH_OK;
  DeviceGuard g(c);
  HIP_OR_FAIL(c, hipHostFree(ptr));
  return ELMH_OK;
}

int elmh_memcpy_h2d_async(elmh_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c) return fail(c, ELMH_ERR_ARG, "null ctx");
  if (bytes && (!dst || !src)) return fail(c, ELMH_ERR_ARG, "null dst/src");
  DeviceGuard g(c);
  if (bytes) HIP_OR_FAIL(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
  return ELMH_OK;
}

int elmh_memcpy_d2h_async(elmh_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c) return fail(c, ELMH_ERR_ARG, "null ctx");
  if (bytes && (!dst || !src)) return fail(c, ELMH_ERR_ARG, "null dst/src");
  DeviceGuard g(c);
  if (bytes) HIP_OR_FAIL(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
  return ELMH_OK;
}

int elmh_memset_dev(elmh_ctx* c, void* dst, int value, size_t bytes) {
  if (!c) return fail(c, ELMH_ERR_ARG, "null ctx");
  if (bytes && !dst) return fail(c, ELMH_ERR_ARG, "null dst");
  DeviceGuard g(c);
  HIP_OR_FAIL(c, launch_fill(dst, value, bytes, c->stream));
  return ELMH_OK;
}

int elmh_rescale_ceiling_dev(elmh_ctx* c, int mode, int blocks, int iters, float* sink, size_t sink_bytes) {
  if (!c || !sink) return fail(c, ELMH_ERR_ARG, "null ctx/sink");
  if (mode < 0 || mode > 2 || blocks < 1 || blocks > 65536 || iters < 1)
    return fail(c, ELMH_ERR_ARG, "rescale ceiling: mode %d, %d workgroups, %d blocks", mode, blocks, iters);
  if (sink_bytes < (size_t)blocks * 256 * sizeof(float))
    return fail(c, ELMH_ERR_ARG, "rescale ceiling: sink of %zu bytes for %d workgroups", sink_bytes, blocks);
  DeviceGuard g(c);
  HIP_OR_FAIL(c, launch_rescale_ceiling(mode, blocks, iters, sink, c->stream));
  return ELMH_OK;
}

size_t elmh_read_sweep_sink_bytes(void) { return read_sweep_sink_bytes(); }

int elmh_read_sweep_dev(elmh_ctx* c, const void* src, size_t bytes, void* sink) {
  if (!c) return fail(c, ELMH_ERR_ARG, "null ctx");
  if (!src || !sink) return fail(c, ELMH_ERR_ARG, "null src/sink");
  if (bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16)
    return fail(c, ELMH_ERR_ARG, "read sweep: src and bytes must be 16-byte aligned (bytes=%zu)", bytes);
  DeviceGuard g(c);
  HIP_OR_FAIL(c, launch_read_sweep(src, bytes, sink, c->stream));
  return ELMH_OK;
}

int elmh_memcpy_d2d(elmh_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c) return fail(c, ELMH_ERR_ARG, "null ctx");
  if (bytes && (!dst || !src)) return fail(c, ELMH_ERR_ARG, "null dst/src");
  DeviceGuard g(c);
  if (bytes) HIP_OR_FAIL(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, c->stream));
  return ELMH_OK;
}

int elmh_argmax_dev(elmh_ctx* c, const float* x, int rows, int64_t n, int32_t* out) {
  if (!c || !x || !out) return fail(c, ELMH_ERR_ARG, "null ctx/x/out");
  if (rows < 1 || n < 1) return fail(c, ELMH_ERR_ARG, "argmax: rows and n must be >= 1 (rows=%d n=%lld)", rows, (long long)n);
  if (n > INT32_MAX) return fail(c, ELMH_ERR_ARG, "argmax: n=%lld exceeds int32 indices", (long long)n);
  DeviceGuard g(c);
  if (rows == 1 && n <= kArgStepMaxN)  // one row (a decode step's logits): over several workgroups
    HIP_OR_FAIL(c, launch_argmax_parts(x, n, out, nullptr, nullptr, 0, c->argmax_scratch, c->stream));
  else
    HIP_OR_FAIL(c, launch_argmax(x, rows, n, out, c->stream));
  return ELMH_OK;
}

int elmh_argmax_step_dev(elmh_ctx* c, const float* x, int64_t n, int32_t* out, int32_t* pos_dev, int32_t* ring,
                         int ring_len) {
  if (!c || !x || !out || !pos_dev || !ring) return fail(c, ELMH_ERR_ARG, "argmax_step: null pointer");
  if (n < 1 || n > kArgStepMaxN)
    return fail(c, ELMH_ERR_ARG, "argmax_step: n=%lld outside 1 .. %d", (long long)n, kArgStepMaxN);
  if (ring_len < 1 || (ring_len & (ring_len - 1)))
    return fail(c, ELMH_ERR_ARG, "argmax_step: ring_len %d is not a power of two", ring_len);
  DeviceGuard g(c);
  HIP_OR_FAIL(c, launch_argmax_parts(x, n, out, pos_dev, ring, ring_len - 1, c->argmax_scratch, c->stream));
  return ELMH_OK;
}

int elmh_embed_dev(elmh_ctx* c, const int32_t* tokens, int T, const elmh_weight* table, float* y) {
  if (!c || !tokens || !table || !y) return fail(c, ELMH_ERR_ARG, "null ctx/tokens/table/y");
  if (T < 1) return fail(c, ELMH_ERR_ARG, "embed: T must be >= 1");
  DeviceGuard g(c);
  HIP_OR_FAIL(c, launch_embed(tokens, T, table->w, y, c->stream));
  return ELMH_OK;
}

int elmh_rmsnorm_dev(elmh_ctx* c, const float* x, const float* w, float* y, int rows, int dim, float eps) {
  if (!c || !x || !w || !y) return fail(c, ELMH_ERR_ARG, "null ctx/x/w/y");
  if (rows < 1 || dim < 1 || dim > 8192) return fail(c, ELMH_ERR_ARG, "rmsnorm: rows %d, dim %d (1 .. 8192)", rows, dim);
  DeviceGuard g(c);
  HIP_OR_FAIL(c, launch_rmsnorm(x, w, y, rows, dim, eps, c->stream));
  return ELMH_OK;
}

int elmh_attention_matmul_dev(elmh_ctx* c, const float* q, const float* k, const float* v, float* out, int T,
                              int pos0, int n_heads, int n_kv, int head_dim, float* k_cache, float* v_cache,
                              int max_ctx, const float* rope_cos, const float* rope_sin, elmh_weight* w, float* y,
                              const float* res, int act, int mode) {
  int rc = check_attention(c, q, k, v, out, T, pos0, n_heads, n_kv, head_dim, k_cache, v_cache, max_ctx, rope_cos,
                           rope_sin);
  if (rc) return rc;
  const int64_t K = (int64_t)n_heads * head_dim;
  elmh_weight* const ws[1] = {w};
  float* const ys[1] = {y};
  const float* const rs[1] = {res};
  if ((rc = check_targets(c, T, K, 1, ws, ys))) return rc;
  if (act < ELMH_ACT_F32 || act > ELMH_ACT_INT8_TOKEN) return fail(c, ELMH_ERR_ARG, "bad act mode %d", act);
  DeviceGuard g(c);
  int8_t* xq = nullptr;
  float* xd = nullptr;
  const int Tpad = (int)round_up(T, kGemmTileT);
  if (T > 1 && head_dim == 64 && block_gemm(T, K, 1, ws, 1, act)) {
    // the GEMM's activation fragments come out of the attention kernel
    ActBufs ab;
    if ((rc = act_buffers(c, Scratch{}, (size_t)Tpad * K, (size_t)Tpad * (K / kBlock) * sizeof(float), 0, &ab)))
      return rc;
    xq = ab.q;
    xd = ab.d;
  }
  bool quantized = false;
  c->attn_fused = 0;
  float* gsc = nullptr;
  if ((rc = attention_scores(c, T, pos0, false, n_heads, head_dim, max_ctx, &gsc))) return rc;
  HIP_OR_FAIL(c, launch_attention(q, k, v, out, T, pos0, nullptr, n_heads, n_kv, head_dim, k_cache, v_cache, max_ctx,
                                  rope_cos, rope_sin, c->stream, xq, xd, Tpad, &quantized, gsc));
  c->attn_fused = quantized ? 1 : 0;
  if (!quantized) return run_matmul(c, out, T, K, 1, ws, ys, res ? rs : nullptr, act, mode);
  for (const auto& grp : by_dtype(1, ws))
    if ((rc = run_gemm_group(c, xq, xd, T, Tpad, K, grp, ws, ys, res ? rs : nullptr, 0, mode == ELMH_FAST))) return rc;
  return ELMH_OK;
}

int elmh_attention_matmul_fused(const elmh_ctx* c) { return c ? c->attn_fused : 0; }

int elmh_attention_dev(elmh_ctx* c, const float* q, const float* k, const float* v, float* out, int T, int pos0,
                       int n_heads, int n_kv, int head_dim, float* k_cache, float* v_cache, int max_ctx,
                       const float* rope_cos, const float* rope_sin) {
  const int rc = check_attention(c, q, k, v, out, T, pos0, n_heads, n_kv, head_dim, k_cache, v_cache, max_ctx,
                                 rope_cos, rope_sin);
  if (rc) return rc;
  DeviceGuard g(c);
  float* gsc = nullptr;
  if (const int r2 = attention_scores(c, T, pos0, false, n_heads, head_dim, max_ctx, &gsc)) return r2;
  HIP_OR_FAIL(c, launch_attention(q, k, v, out, T, pos0, nullptr, n_heads, n_kv, head_dim, k_cache, v_cache, max_ctx,
                                  rope_cos, rope_sin, c->stream, nullptr, nullptr, 0, nullptr, gsc));
  return ELMH_OK;
}

int elmh_attention_step_supported(int head_dim, int max_ctx) {
  return head_dim >= 4 && head_dim % 4 == 0 && head_dim <= 256 && max_ctx >= 1;
}

int elmh_attention_step_dev(elmh_ctx* c, const float* q, const float* k, const float* v, float* out,
                            const int32_t* pos_dev, int n_heads, int n_kv, int head_dim, float* k_cache, float* v_cache,
                            int max_ctx, const float* rope_cos, const float* rope_sin) {
  if (!c || !q || !k || !v || !out || !pos_dev || !k_cache || !v_cache)
    return fail(c, ELMH_ERR_ARG, "attention_step: null pointer");
  if (max_ctx < 1 || n_heads < 1 || n_kv < 1 || n_heads % n_kv || head_dim < 4 || head_dim % 4 || head_dim > 256)
    return fail(c, ELMH_ERR_ARG, "attention_step: heads %d / kv heads %d / head_dim %d / max_ctx %d", n_heads, n_kv,
                head_dim, max_ctx);
  if (!rope_cos != !rope_sin) return fail(c, ELMH_ERR_ARG, "attention_step: rope_cos and rope_sin go together");
  DeviceGuard g(c);
  float* gsc = nullptr;
  if (const int rc = attention_scores(c, 1, 0, true, n_heads, head_dim, max_ctx, &gsc)) return rc;
  HIP_OR_FAIL(c, launch_attention(q, k, v, out, 1, 0, pos_dev, n_heads, n_kv, head_dim, k_cache, v_cache, max_ctx,
                                  rope_cos, rope_sin, c->stream, nullptr, nullptr, 0, nullptr, gsc));
  return ELMH_OK;
}

int elmh_synchronize(elmh_ctx* c) {
  if (!c) return fail(c, ELMH_ERR_ARG, "null ctx");
  DeviceGuard g(c);
  HIP_OR_FAIL(c, hipStreamSynchronize(c->stream));
  return ELMH_OK;
}

void* elmh_stream(elmh_ctx* c) { return c ? (void*)c->stream : nullptr; }

int elmh_event_create(elmh_ctx* c, void** ev) {
  if (!c || !ev) return fail(c, ELMH_ERR_ARG, "null argument");
  DeviceGuard g(c);
  HIP_OR_FAIL(c, hipEventCreate((hipEvent_t*)ev));
  return ELMH_OK;
}

int elmh_event_destroy(elmh_ctx* c, void* ev) {
  if (!c) return fail(c, ELMH_ERR_ARG, "null ctx");
  DeviceGuard g(c);
  if (ev) HIP_OR_FAIL(c, hipEventDestroy((hipEvent_t)ev));
  return ELMH_OK;
}

int elmh_event_record(elmh_ctx* c, void* ev) {
  if (!c || !ev) return fail(c, ELMH_ERR_ARG, "null argument");
  DeviceGuard g(c);
  HIP_OR_FAIL(c, hipEventRecord((hipEvent_t)ev, c->stream));
  return ELMH_OK;
}

int elmh_event_elapsed(elmh_ctx* c, void* a, void* b, float* ms) {
  if (!c || !a || !b || !ms) return fail(c, ELMH_ERR_ARG, "null argument");
  DeviceGuard g(c);
  HIP_OR_FAIL(c, hipEventSynchronize((hipEvent_t)b));
  HIP_OR_FAIL(c, hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
  return ELMH_OK;
}

int elmh_graph_begin(elmh_ctx* c) {
  if (!c) return fail(c, ELMH_ERR_ARG, "null ctx");
  DeviceGuard g(c);
  HIP_OR_FAIL(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
  return ELMH_OK;
}

int elmh_graph_end(elmh_ctx* c, void** exec) {
  if (!c || !exec) return fail(c, ELMH_ERR_ARG, "null argument");
  DeviceGuard g(c);
  hipGraph_t graph = nullptr;
  HIP_OR_FAIL(c, hipStreamEndCapture(c->stream, &graph));
  hipGraphExec_t ge = nullptr;
  hipError_t e = hipGraphInstantiate(&ge, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (e != hipSuccess) return fail(c, ELMH_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
  *exec = ge;
  return ELMH_OK;
}

int elmh_graph_launch(elmh_ctx* c, void* exec) {
  if (!c || !exec) return fail(c, ELMH_ERR_ARG, "null argument");
  DeviceGuard g(c);
  HIP_OR_FAIL(c, hipGraphLaunch((hipGraphExec_t)exec, c->stream));
  return ELMH_OK;
}

int elmh_graph_destroy(elmh_ctx* c, void* exec) {
  if (!c) return fail(c, ELMH_ERR_ARG, "null ctx");
  DeviceGuard g(c);
  if (exec) HIP_OR_FAIL(c, hipGraphExecDestroy((hipGraphExec_t)exec));
  return ELMH_OK;
}

}  // extern "C"

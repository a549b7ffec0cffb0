// TEST INFRASTRUCTURE ONLY — extern "C" wrappers around edgelm's own C++ (compiled from the
// reference sources by oracle/Makefile into oracle/_ref/libedgelm_ref.so). Used to pin the C
// oracle, to generate fixtures, and as bench.py's cpu_baseline ("kind": "reference"). The
// product never links or loads it.
#include <algorithm>
#include <chrono>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "edgelm/backend.hpp"
#include "edgelm/kernels.hpp"
#include "edgelm/model.hpp"
#include "edgelm/runtime.hpp"
#include "edgelm/thread_pool.hpp"
#include "edgelm/tokenizer.hpp"

using namespace edgelm;

namespace {

Tensor make_tensor(int dtype, int64_t rows, int64_t cols, const void* data, const float* scales) {
  Tensor t;
  t.kind = TensorKind::Weight;
  t.dtype = static_cast<DType>(dtype);
  t.rows = rows;
  t.cols = cols;
  t.data = data;
  t.scales = scales;
  t.group = dtype == 2 ? 32 : dtype == 1 ? static_cast<int>(cols) : 0;
  return t;
}

struct Pool {
  ThreadPool pool;
  std::vector<std::vector<float>> bufs;
  std::vector<float*> ptrs;
  Pool(int threads, int T, int64_t max_k) : pool(threads) {
    for (int i = 0; i < pool.size(); ++i) bufs.emplace_back(cpu::scratch_floats(T, max_k, 1, 1));
    for (auto& b : bufs) ptrs.push_back(b.data());
  }
};

thread_local std::string g_err;

}  // namespace

extern "C" {

const char* eref_last_error() { return g_err.c_str(); }

void eref_quantize_q8(const float* w, int64_t n, int64_t k, int8_t* out, float* scales) { quantize_q8(w, n, k, out, scales); }
void eref_quantize_q4(const float* w, int64_t n, int64_t k, uint8_t* out, float* scales) { quantize_q4(w, n, k, out, scales); }
void eref_dequantize_row(int dtype, int64_t rows, int64_t cols, const void* data, const float* scales, int64_t row,
                         float* out) {
  Tensor t = make_tensor(dtype, rows, cols, data, scales);
  dequantize_row(t, row, out);
}
void eref_quantize_act_row(const float* x, int64_t k, int8_t* q, float* d) { quantize_act_row(x, k, q, d); }

void eref_ref_matmul(const float* x, int T, int dtype, int64_t rows, int64_t cols, const void* data, const float* scales,
                     float* y, const float* residual, int act_quant) {
  Tensor t = make_tensor(dtype, rows, cols, data, scales);
  ref::matmul(x, T, t, y, residual, act_quant != 0);
}

void eref_ref_swiglu(const float* x, int T, int dtype_g, int dtype_u, int64_t rows, int64_t cols, const void* dg,
                     const float* sg, const void* du, const float* su, float* y, int act_quant) {
  Tensor g = make_tensor(dtype_g, rows, cols, dg, sg), u = make_tensor(dtype_u, rows, cols, du, su);
  ref::swiglu(x, T, g, u, y, act_quant != 0);
}

void eref_set_simd(int on) { cpu::set_simd(on != 0); }

void* eref_pool_create(int threads, int max_T, int64_t max_k) { return new Pool(threads, max_T, max_k); }
void eref_pool_destroy(void* p) { delete static_cast<Pool*>(p); }

// cpu::matmul over n targets. dtypes/rows/data/scales/y/residual are arrays of length n.
int eref_cpu_matmul(void* pool, const float* x, int T, int n, const int* dtypes, const int64_t* rows, int64_t cols,
                    const void* const* data, const float* const* scales, float* const* y, const float* const* residual,
                    int act_quant) {
  try {
    Pool* p = static_cast<Pool*>(pool);
    std::vector<Tensor> ts;
    for (int i = 0; i < n; ++i) ts.push_back(make_tensor(dtypes[i], rows[i], cols, data[i], scales[i]));
    std::vector<MatmulTarget> tg;
    for (int i = 0; i < n; ++i) tg.push_back({&ts[i], y[i], residual ? residual[i] : nullptr});
    std::vector<int8_t> q(static_cast<size_t>(T) * cols);
    std::vector<float> d(static_cast<size_t>(T) * (cols / kActBlock + 1));
    ActBuf aq{q.data(), d.data()};
    cpu::matmul(x, T, tg, &p->pool, p->ptrs.data(), act_quant ? &aq : nullptr);
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return 1;
  }
}

int eref_cpu_swiglu(void* pool, const float* x, int T, int dtype_g, int dtype_u, int64_t rows, int64_t cols,
                    const void* dg, const float* sg, const void* du, const float* su, float* y, int act_quant) {
  try {
    Pool* p = static_cast<Pool*>(pool);
    Tensor g = make_tensor(dtype_g, rows, cols, dg, sg), u = make_tensor(dtype_u, rows, cols, du, su);
    std::vector<int8_t> q(static_cast<size_t>(T) * cols);
    std::vector<float> d(static_cast<size_t>(T) * (cols / kActBlock + 1));
    ActBuf aq{q.data(), d.data()};
    cpu::swiglu(x, T, g, u, y, &p->pool, p->ptrs.data(), act_quant ? &aq : nullptr);
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return 1;
  }
}

// ---- whole-model runs through the reference's own loader, passes, partitioner and Session ----

struct RefRun {
  Model model;
  std::unique_ptr<Session> session;
};

// Loads an .elm file and builds a Session. backends: comma-separated preference list.
void* eref_session_create(const char* path, const char* backends, int threads, int max_ctx, int max_batch,
                          int all_logits, int act_quant, int fuse) {
  try {
    auto r = std::make_unique<RefRun>();
    r->model = Model::load(path);
    SessionOptions o;
    o.backends.clear();
    std::string s(backends);
    size_t pos = 0;
    while (pos <= s.size()) {
      const size_t c = s.find(',', pos);
      const std::string b = s.substr(pos, c == std::string::npos ? std::string::npos : c - pos);
      if (!b.empty()) o.backends.push_back(b);
      if (c == std::string::npos) break;
      pos = c + 1;
    }
    o.threads = threads;
    o.max_ctx = max_ctx;
    o.max_batch = max_batch;
    o.all_logits = all_logits != 0;
    o.act_quant = act_quant != 0;
    o.fuse = fuse != 0;
    r->session = std::make_unique<Session>(r->model, o);
    return r.release();
  } catch (const std::exception& e) {
    g_err = e.what();
    return nullptr;
  }
}

void eref_session_destroy(void* h) { delete static_cast<RefRun*>(h); }
void eref_session_reset(void* h) { static_cast<RefRun*>(h)->session->reset(); }
int eref_session_vocab(void* h) { return static_cast<RefRun*>(h)->model.cfg.vocab; }

// forward(tokens, n); copies rows*vocab logits into out (rows = all_logits ? n : 1).
int eref_session_forward(void* h, const int32_t* tokens, int n, float* out) {
  try {
    RefRun* r = static_cast<RefRun*>(h);
    const float* lg = r->session->forward(tokens, n, n > 1 ? "prefill" : "decode");
    const int rows = r->session->options().all_logits ? n : 1;
    std::memcpy(out, lg, sizeof(float) * static_cast<size_t>(rows) * r->model.cfg.vocab);
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return 1;
  }
}

int32_t eref_argmax(const float* logits, int n) { return argmax(logits, n); }

// The bench protocol of bench.py on edgelm's own Session, timed here in C: reset, prefill (edgelm's
// Session::prefill in max_batch chunks) and argmax of the last logits row (TTFT), `warmup` untimed
// greedy decode steps, then `steps` timed ones (edgelm's argmax, tokenizer.cpp:187-189).
int eref_session_bench(void* h, const int32_t* prompt, int n_prompt, int warmup, int steps, double* ttft_ms,
                       double* decode_ms, int32_t* tokens_out) {
  try {
    RefRun* r = static_cast<RefRun*>(h);
    Session& s = *r->session;
    const int V = r->model.cfg.vocab;
    auto last_row = [&](const float* lg, int n) { return s.options().all_logits ? lg + static_cast<size_t>(n - 1) * V : lg; };
    s.reset();
    const auto t0 = std::chrono::steady_clock::now();
    const float* lg = s.prefill(std::vector<int32_t>(prompt, prompt + n_prompt));
    const int mb = s.options().max_batch, tail = n_prompt % mb ? n_prompt % mb : mb;
    int32_t tok = argmax(last_row(lg, tail), V);
    const auto t1 = std::chrono::steady_clock::now();
    if (tokens_out) tokens_out[0] = tok;
    for (int i = 0; i < warmup; ++i) {
      tok = argmax(last_row(s.decode(tok), 1), V);
      if (tokens_out) tokens_out[1 + i] = tok;
    }
    const auto t2 = std::chrono::steady_clock::now();
    for (int i = 0; i < steps; ++i) {
      tok = argmax(last_row(s.decode(tok), 1), V);
      if (tokens_out) tokens_out[1 + warmup + i] = tok;
    }
    const auto t3 = std::chrono::steady_clock::now();
    *ttft_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    *decode_ms = std::chrono::duration<double, std::milli>(t3 - t2).count();
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return 1;
  }
}

// edgelm's Model::load then convert_weights(dtype) (model.cpp:220-251); copies weight `name` into data /
// scales (capacities in, sizes out) and returns its dtype, or -1.
int eref_convert_weight(const char* path, int dtype, const char* name, void* data, int64_t* data_bytes, void* scales,
                        int64_t* scale_bytes) {
  try {
    Model m = Model::load(path);
    m.convert_weights(static_cast<DType>(dtype));
    for (const Tensor& t : m.graph.tensors) {
      if (!t.is_weight() || t.name != name) continue;
      if (static_cast<int64_t>(t.data_bytes) > *data_bytes || static_cast<int64_t>(t.scale_bytes) > *scale_bytes) {
        g_err = "buffer too small";
        return -1;
      }
      std::memcpy(data, t.data, t.data_bytes);
      if (t.scale_bytes) std::memcpy(scales, t.scales, t.scale_bytes);
      *data_bytes = static_cast<int64_t>(t.data_bytes);
      *scale_bytes = static_cast<int64_t>(t.scale_bytes);
      return static_cast<int>(t.dtype);
    }
    g_err = std::string("no weight ") + name;
    return -1;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

// describe_partitions of the session's graph (for partition-count parity tests)
int eref_session_describe(void* h, char* buf, int cap) {
  RefRun* r = static_cast<RefRun*>(h);
  const std::string s = describe_partitions(r->session->graph(), r->session->partitions());
  std::strncpy(buf, s.c_str(), static_cast<size_t>(cap) - 1);
  buf[cap - 1] = 0;
  return static_cast<int>(r->session->graph().ops.size());
}


// RopeTable (kernels_ref.cpp:11-21), cpu::rmsnorm (kernels_cpu.cpp:326-335) and cpu::attention
// (kernels_cpu.cpp:417-488) as edgelm runs them (no pool: serial).
void eref_rope_table(int head_dim, int max_pos, float theta, float* cos_out, float* sin_out) {
  RopeTable rt(head_dim, max_pos, theta);
  std::memcpy(cos_out, rt.cos.data(), rt.cos.size() * sizeof(float));
  std::memcpy(sin_out, rt.sin.data(), rt.sin.size() * sizeof(float));
}
void eref_rmsnorm(const float* x, const float* w, float* y, int rows, int dim, float eps) {
  cpu::rmsnorm(x, w, y, rows, dim, eps, nullptr);
}
void eref_attention(const float* q, const float* k, const float* v, float* out, int T, int pos0, int n_heads, int n_kv,
                    int hd, float* kc, float* vc, int max_ctx, int rope, float theta) {
  RopeTable rt(hd, max_ctx, theta);
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.T = T;
  a.pos0 = pos0;
  a.n_heads = n_heads;
  a.n_kv = n_kv;
  a.head_dim = hd;
  a.cache.k = kc;
  a.cache.v = vc;
  a.cache.max_ctx = max_ctx;
  a.rope = rope ? &rt : nullptr;
  std::vector<float> scratch(static_cast<size_t>(max_ctx) + hd + 16);
  float* sp = scratch.data();
  cpu::attention(a, nullptr, &sp);
}
}  // extern "C"

// edgelm's reference-backend ops (kernels_ref.cpp:41-57,82-151), serial.
extern "C" {
void eref_ref_rmsnorm(const float* x, const float* w, float* y, int rows, int dim, float eps) {
  ref::rmsnorm(x, w, y, rows, dim, eps);
}
void eref_ref_attention(const float* q, const float* k, const float* v, float* out, int T, int pos0, int n_heads,
                        int n_kv, int hd, float* kc, float* vc, int max_ctx, int rope, float theta) {
  RopeTable rt(hd, max_ctx, theta);
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.T = T;
  a.pos0 = pos0;
  a.n_heads = n_heads;
  a.n_kv = n_kv;
  a.head_dim = hd;
  a.cache.k = kc;
  a.cache.v = vc;
  a.cache.max_ctx = max_ctx;
  a.rope = rope ? &rt : nullptr;
  ref::attention(a);
}
void eref_ref_rope(const float* x, float* y, int T, int n_heads, int hd, int pos0, int max_pos, float theta) {
  RopeTable rt(hd, max_pos, theta);
  ref::rope(x, y, T, n_heads, hd, pos0, rt);
}
void eref_ref_elementwise(int op, const float* a, const float* b, float* y, int64_t n) {
  if (op == 0) ref::add(a, b, y, n);
  else if (op == 1) ref::mul(a, b, y, n);
  else ref::silu(a, y, n);
}
// cpu::attention over a pool of `threads` (scratch per thread as the cpu backend sizes it)
void eref_cpu_attention_pool(const float* q, const float* k, const float* v, float* out, int T, int pos0, int n_heads,
                             int n_kv, int hd, float* kc, float* vc, int max_ctx, int rope, float theta, int threads) {
  RopeTable rt(hd, max_ctx, theta);
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.T = T;
  a.pos0 = pos0;
  a.n_heads = n_heads;
  a.n_kv = n_kv;
  a.head_dim = hd;
  a.cache.k = kc;
  a.cache.v = vc;
  a.cache.max_ctx = max_ctx;
  a.rope = rope ? &rt : nullptr;
  ThreadPool pool(threads);
  std::vector<std::vector<float>> bufs;
  std::vector<float*> ptrs;
  for (int i = 0; i < pool.size(); ++i) bufs.emplace_back(cpu::scratch_floats(T, hd, max_ctx, hd));
  for (auto& b : bufs) ptrs.push_back(b.data());
  cpu::attention(a, &pool, ptrs.data());
}
}  // extern "C"

// ---- CPU baseline of the matmul family: edgelm's cpu::matmul / cpu::swiglu (kernels_cpu.cpp:339-411) on its
// own ThreadPool (thread_pool.cpp:31-63, dynamic chunking), timed here in C as edgelm's bench times a
// step (main.cpp:199-217): `warm` untimed calls, then calls until `budget_s` seconds have passed (at least
// `min_reps`, at most `max_reps`); the median call time goes to *median_ms, the count to *reps.
// op 0: MATMUL / MATMUL_N / MATMUL_ADD over n targets (residual may be null); op 1: FFN_SWIGLU of targets
// 0 (gate) and 1 (up) into y[0].
extern "C" int eref_time_cpu_op(int op, int threads, const float* x, int T, int n, const int* dtypes,
                                const int64_t* rows, int64_t cols, const void* const* data,
                                const float* const* scales, float* const* y, const float* const* residual,
                                int act_quant, int warm, int min_reps, int max_reps, double budget_s,
                                double* median_ms, int* reps) {
  try {
    Pool p(threads, T, cols);
    std::vector<Tensor> ts;
    for (int i = 0; i < n; ++i) ts.push_back(make_tensor(dtypes[i], rows[i], cols, data[i], scales[i]));
    std::vector<MatmulTarget> tg;
    for (int i = 0; i < n; ++i) tg.push_back({&ts[i], y[i], residual ? residual[i] : nullptr});
    std::vector<int8_t> q(static_cast<size_t>(T) * cols);
    std::vector<float> d(static_cast<size_t>(T) * (cols / kActBlock + 1));
    ActBuf aq{q.data(), d.data()};
    const ActBuf* a = act_quant ? &aq : nullptr;
    auto call = [&] {
      if (op == 1) cpu::swiglu(x, T, ts[0], ts[1], y[0], &p.pool, p.ptrs.data(), a);
      else cpu::matmul(x, T, tg, &p.pool, p.ptrs.data(), a);
    };
    for (int i = 0; i < warm; ++i) call();
    std::vector<double> ms;
    const auto t_end = std::chrono::steady_clock::now() + std::chrono::duration<double>(budget_s);
    while (static_cast<int>(ms.size()) < max_reps &&
           (static_cast<int>(ms.size()) < min_reps || std::chrono::steady_clock::now() < t_end)) {
      const auto t0 = std::chrono::steady_clock::now();
      call();
      ms.push_back(std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count());
    }
    std::sort(ms.begin(), ms.end());
    *median_ms = ms[ms.size() / 2];
    *reps = static_cast<int>(ms.size());
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return 1;
  }
}

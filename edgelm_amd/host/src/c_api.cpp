// C API of the host library (include/edgelm_host.h) for callers that are not C++.
#include <chrono>
#include <cstring>
#include <string>

#include "edgelm/runtime.hpp"
#include "edgelm_host.h"

using namespace edgelm;

namespace edgelm {
void write_random_model(const std::string& path, const elm_model_spec& spec);  // elm_synth.cpp
}

struct elm_model {
  Model m;
};
struct elm_session {
  std::unique_ptr<Session> s;
};

namespace {
thread_local std::string g_err;

std::vector<std::string> split(const char* csv) {
  std::vector<std::string> out;
  std::string cur;
  for (const char* p = csv ? csv : ""; *p; ++p) {
    if (*p == ',') {
      if (!cur.empty()) out.push_back(cur);
      cur.clear();
    } else {
      cur += *p;
    }
  }
  if (!cur.empty()) out.push_back(cur);
  return out;
}

template <class F>
int guard(F&& f) {
  try {
    return f();
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

void copy_text(const std::string& s, char* buf, int cap) {
  if (!buf || cap <= 0) return;
  std::strncpy(buf, s.c_str(), static_cast<size_t>(cap) - 1);
  buf[cap - 1] = 0;
}

double ms_between(std::chrono::steady_clock::time_point a, std::chrono::steady_clock::time_point b) {
  return std::chrono::duration<double, std::milli>(b - a).count();
}
}  // namespace

extern "C" {

const char* elm_last_error(void) { return g_err.c_str(); }

elm_model* elm_model_load(const char* path) {
  try {
    auto* m = new elm_model{Model::load(path)};
    return m;
  } catch (const std::exception& e) {
    g_err = e.what();
    return nullptr;
  }
}

void elm_model_free(elm_model* m) { delete m; }

int elm_model_convert(elm_model* m, int dtype, int threads) {
  return guard([&] {
    if (!m) throw std::runtime_error("edgelm: null model");
    if (dtype < 0 || dtype > 2) throw std::runtime_error("edgelm: convert to f32 (0), q8 (1) or q4 (2)");
    m->m.convert_weights(static_cast<DType>(dtype), threads);
    return 0;
  });
}

int elm_model_prefault(const elm_model* m) {
  return guard([&] {
    if (!m) throw std::runtime_error("edgelm: null model");
    m->m.prefault();
    return 0;
  });
}

int elm_model_write_device_image(const elm_model* m, const char* path, int threads) {
  return guard([&] {
    if (!m || !path) throw std::runtime_error("edgelm: null argument");
    return m->m.write_device_image(path, threads);
  });
}

int elm_model_attach_device_image(elm_model* m, const char* path) {
  return guard([&] {
    if (!m || !path) throw std::runtime_error("edgelm: null argument");
    return m->m.attach_device_image(path) ? 1 : 0;
  });
}

int elm_model_weight(const elm_model* m, const char* name, int64_t* rows, int64_t* cols, void* data, float* scales) {
  return guard([&] {
    if (!m || !name) throw std::runtime_error("edgelm: null argument");
    for (const Tensor& t : m->m.graph.tensors) {
      if (!t.is_weight() || t.name != name) continue;
      if (rows) *rows = t.rows;
      if (cols) *cols = t.cols;
      if (data) std::memcpy(data, t.data, t.data_bytes);
      if (scales && t.scales) std::memcpy(scales, t.scales, t.scale_bytes);
      return static_cast<int>(t.dtype);
    }
    return -1;
  });
}

int elm_write_random_model(const char* path, const elm_model_spec* spec) {
  return guard([&] {
    if (!path || !spec) throw std::runtime_error("edgelm: null argument");
    write_random_model(path, *spec);
    return 0;
  });
}

int elm_model_config(const elm_model* m, int* o) {
  if (!m || !o) return -1;
  const Config& c = m->m.cfg;
  const int v[10] = {c.vocab, c.dim, c.hidden, c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim, c.max_seq,
                     static_cast<int>(c.weight_dtype), c.tied ? 1 : 0};
  std::memcpy(o, v, sizeof v);
  return 0;
}

int elm_model_fusion(const elm_model* m, int* o) {
  return guard([&] {
    Graph g = m->m.graph;
    const FusionStats s = optimize(g);
    const int v[6] = {s.swiglu, s.shared_input, s.residual, s.rope, static_cast<int>(s.ops_before),
                      static_cast<int>(s.ops_after)};
    std::memcpy(o, v, sizeof v);
    return 0;
  });
}

int elm_model_plan(const elm_model* m, int fuse, int T, int L, int64_t* arena, int64_t* naive) {
  return guard([&] {
    Graph g = m->m.graph;
    if (fuse) optimize(g);
    const MemoryPlan p = plan_memory(g, T, L);
    *arena = static_cast<int64_t>(p.arena_bytes);
    *naive = static_cast<int64_t>(p.naive_bytes);
    return plan_is_valid(p) ? 1 : 0;
  });
}

int elm_model_partition(const elm_model* m, const char* backends, int fuse, char* buf, int cap) {
  return guard([&] {
    Graph g = m->m.graph;
    if (fuse) optimize(g);
    std::vector<std::unique_ptr<Backend>> owned;
    for (const std::string& b : split(backends)) {
      if (b == "reference" || b == "ref") continue;
      owned.push_back(b == "hip" || b == "hip-matmul" ? make_hip_planning_backend(b == "hip") : make_backend(b));
    }
    owned.push_back(make_reference_backend());
    std::vector<Backend*> pref;
    for (auto& b : owned) pref.push_back(b.get());
    const auto parts = partition_graph(g, pref);
    copy_text(describe_partitions(g, parts), buf, cap);
    return static_cast<int>(parts.size());
  });
}

elm_session* elm_session_create(const elm_model* m, const char* backends, int threads, int max_ctx, int max_batch,
                                int all_logits, int act_quant, int fuse) {
  try {
    SessionOptions o;
    o.backends = split(backends);
    o.threads = threads;
    o.max_ctx = max_ctx;
    o.max_batch = max_batch;
    o.all_logits = all_logits != 0;
    o.act_quant = act_quant != 0;
    o.fuse = fuse != 0;
    auto* s = new elm_session{std::make_unique<Session>(m->m, o)};
    return s;
  } catch (const std::exception& e) {
    g_err = e.what();
    return nullptr;
  }
}

void elm_session_destroy(elm_session* s) { delete s; }

int elm_session_forward(elm_session* s, const int32_t* tokens, int n, float* out) {
  return guard([&] {
    const float* lg = s->s->forward(tokens, n);
    const int rows = s->s->options().all_logits ? n : 1;
    if (out) std::memcpy(out, lg, sizeof(float) * static_cast<size_t>(rows) * s->s->vocab());
    return 0;
  });
}

int elm_session_prefill(elm_session* s, const int32_t* tokens, int n, float* out) {
  return guard([&] {
    const float* lg = s->s->prefill(std::vector<int32_t>(tokens, tokens + n));
    const int mb = s->s->options().max_batch;
    const int last = n % mb ? n % mb : mb;
    const int rows = s->s->options().all_logits ? last : 1;
    if (out) std::memcpy(out, lg, sizeof(float) * static_cast<size_t>(rows) * s->s->vocab());
    return 0;
  });
}

int elm_session_reset(elm_session* s) {
  s->s->reset();
  return 0;
}

int elm_session_pos(const elm_session* s) { return s->s->pos(); }

int elm_session_describe(const elm_session* s, char* buf, int cap) {
  copy_text(describe_partitions(s->s->graph(), s->s->partitions()), buf, cap);
  return static_cast<int>(s->s->graph().ops.size());
}

int elm_session_greedy(elm_session* s, const int32_t* tokens, int n, int32_t* next) {
  return guard([&] {
    if (!s || !tokens || n < 1 || !next) throw std::runtime_error("edgelm: bad greedy arguments");
    *next = s->s->greedy(tokens, n);
    return 0;
  });
}

int elm_session_greedy_steps(elm_session* s, int32_t first, int n, int32_t* tokens) {
  return guard([&] {
    if (!s || n < 1 || !tokens) throw std::runtime_error("edgelm: bad greedy_steps arguments");
    s->s->greedy_steps(first, n, tokens);
    return 0;
  });
}

int elm_session_bench(elm_session* s, const int32_t* prompt, int n_prompt, int warmup, int steps, double* ttft_ms,
                      double* decode_ms, int32_t* tokens_out) {
  return guard([&] {
    if (!s || !prompt || n_prompt < 1 || warmup < 0 || steps < 1) throw std::runtime_error("edgelm: bad bench arguments");
    Session& ss = *s->s;
    ss.reset();
    const auto t0 = std::chrono::steady_clock::now();
    int32_t tok = ss.greedy_prefill(std::vector<int32_t>(prompt, prompt + n_prompt));
    const auto t1 = std::chrono::steady_clock::now();
    if (tokens_out) tokens_out[0] = tok;
    if (warmup > 0) tok = ss.greedy_steps(tok, warmup, tokens_out ? tokens_out + 1 : nullptr);
    // greedy_steps returns with every step's token id on the host, so the clock brackets finished work
    const auto t2 = std::chrono::steady_clock::now();
    tok = ss.greedy_steps(tok, steps, tokens_out ? tokens_out + 1 + warmup : nullptr);
    const auto t3 = std::chrono::steady_clock::now();
    *ttft_ms = ms_between(t0, t1);
    *decode_ms = ms_between(t2, t3);
    return 0;
  });
}

int elm_session_generate(elm_session* s, const int32_t* prompt, int n_prompt, int gen, double* prefill_ms,
                         double* ttft_ms, double* decode_ms, int32_t* tokens_out) {
  return guard([&] {
    Session& ss = *s->s;
    ss.reset();
    const auto t0 = std::chrono::steady_clock::now();
    // greedy steps take the argmax where the logits are (the device, for a hip output), so the
    // prefill and the first argmax are timed together: both are in TTFT
    int32_t tok = ss.greedy_prefill(std::vector<int32_t>(prompt, prompt + n_prompt));
    const auto t1 = std::chrono::steady_clock::now();
    const auto t2 = t1;
    if (tokens_out) tokens_out[0] = tok;
    if (gen > 0) tok = ss.greedy_steps(tok, gen, tokens_out ? tokens_out + 1 : nullptr);
    const auto t3 = std::chrono::steady_clock::now();
    *prefill_ms = ms_between(t0, t1);
    *ttft_ms = ms_between(t0, t2);
    *decode_ms = ms_between(t2, t3);
    return 0;
  });
}

}  // extern "C"

// ---- the host ops alone (test hooks): flavor 0 = edgelm's reference backend, 1 = its cpu backend
#include "edgelm/host_ops.hpp"

namespace {
host::Flavor flavor_of(int f) { return f ? host::Flavor::Cpu : host::Flavor::Reference; }
}  // namespace

extern "C" int elm_host_rope_table(int head_dim, int max_pos, float theta, float* cos_out, float* sin_out) {
  return guard([&] {
    const RopeTable rt(head_dim, max_pos, theta);
    std::memcpy(cos_out, rt.cos.data(), rt.cos.size() * sizeof(float));
    std::memcpy(sin_out, rt.sin.data(), rt.sin.size() * sizeof(float));
    return 0;
  });
}

extern "C" int elm_host_rmsnorm(const float* x, const float* w, float* y, int rows, int dim, float eps, int flavor,
                                int threads) {
  return guard([&] {
    ThreadPool pool(threads);
    host::rmsnorm(x, w, y, rows, dim, eps, flavor_of(flavor), threads > 1 ? &pool : nullptr);
    return 0;
  });
}

extern "C" int elm_host_attention(const float* q, const float* k, const float* v, float* out, int T, int pos0,
                                  int n_heads, int n_kv, int head_dim, float* kc, float* vc, int max_ctx, int rope,
                                  float theta, int flavor, int threads) {
  return guard([&] {
    const RopeTable rt(head_dim, max_ctx, theta);
    AttnArgs a{q, k, v, out, T, pos0, n_heads, n_kv, head_dim, KVLayer{kc, vc, max_ctx}, rope ? &rt : nullptr};
    ThreadPool pool(threads);
    host::attention(a, flavor_of(flavor), threads > 1 ? &pool : nullptr);
    return 0;
  });
}

extern "C" int elm_host_rope(const float* x, float* y, int T, int n_heads, int head_dim, int pos0, int max_pos,
                             float theta) {
  return guard([&] {
    const RopeTable rt(head_dim, max_pos, theta);
    host::rope(x, y, T, n_heads, head_dim, pos0, rt);
    return 0;
  });
}

// op: 0 add, 1 mul, 2 silu (b unused)
extern "C" int elm_host_elementwise(int op, const float* a, const float* b, float* y, int64_t n) {
  return guard([&] {
    if (op == 0) host::add(a, b, y, n);
    else if (op == 1) host::mul(a, b, y, n);
    else host::silu(a, y, n);
    return 0;
  });
}

// Thread pool and the host-side non-matmul ops (see host_ops.hpp).
#include "edgelm/host_ops.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

#include "edgelm/model.hpp"

namespace edgelm {

// ------------------------------------------------------------------ thread pool

namespace {
inline void relax() {
#if defined(__x86_64__) || defined(__i386__)
  __builtin_ia32_pause();
#endif
}
constexpr int kSpin = 100000;
}  // namespace

ThreadPool::ThreadPool(int threads) : n_(std::max(1, threads)), slots_(static_cast<size_t>(std::max(1, threads))) {
  for (int i = 1; i < n_; ++i) threads_.emplace_back([this, i] { worker(i); });
}

ThreadPool::~ThreadPool() {
  stop_.store(true);
  {
    std::lock_guard<std::mutex> lk(mu_);
    for (Slot& s : slots_) s.epoch.fetch_add(1);
  }
  cv_.notify_all();
  for (std::thread& t : threads_) t.join();
}

void ThreadPool::worker(int id) {
  Slot& me = slots_[static_cast<size_t>(id)];
  uint64_t seen = 0;
  for (;;) {
    int spins = 0;
    while (me.epoch.load(std::memory_order_acquire) == seen && spins < kSpin) {
      relax();
      ++spins;
    }
    if (me.epoch.load(std::memory_order_acquire) == seen) {
      std::unique_lock<std::mutex> lk(mu_);
      sleepers_.fetch_add(1);
      cv_.wait(lk, [&] { return me.epoch.load(std::memory_order_acquire) != seen; });
      sleepers_.fetch_sub(1);
    }
    if (stop_.load()) return;
    seen = me.epoch.load(std::memory_order_acquire);
    // the job (fn_, items_) stays untouched until every worker has published `done`
    const int64_t b = items_ * id / n_, e = items_ * (id + 1) / n_;
    if (b < e) (*fn_)(b, e);
    me.done.store(seen, std::memory_order_release);
  }
}

void ThreadPool::parallel_for(int64_t n, const std::function<void(int64_t, int64_t)>& fn) {
  if (n <= 0) return;
  if (n_ == 1 || n == 1) {
    fn(0, n);
    return;
  }
  fn_ = &fn;
  items_ = n;
  const uint64_t ep = ++epoch_;
  for (int i = 1; i < n_; ++i) slots_[static_cast<size_t>(i)].epoch.store(ep);  // seq_cst: ordered before the sleepers check
  if (sleepers_.load() > 0) {
    std::lock_guard<std::mutex> lk(mu_);
    cv_.notify_all();
  }
  const int64_t e0 = n / n_;
  if (e0 > 0) fn(0, e0);
  for (int i = 1; i < n_; ++i)
    while (slots_[static_cast<size_t>(i)].done.load(std::memory_order_acquire) != ep) relax();
}

// ------------------------------------------------------------------ ops
//
// The float arithmetic below is edgelm's, operation for operation, so that sessions mixing these
// host ops with the hip backend are bit-identical to edgelm's. The two edgelm host backends differ in
// two accumulation choices only, named here as a Flavor:
//   * a dot product or sum of squares: one running sum (reference backend, kernels_ref.cpp:41-57,
//     100-141) or four running sums over the element index mod 4, the tail added to the first, and
//     the four combined as (0 + 1) + (2 + 3) (cpu backend, kernels_cpu.cpp:32-43, 326-335, 417-488);
//   * the softmax weight of a position: e / sum (reference) or e * (1 / sum) (cpu).
// Every other rounding (RoPE's rotation, the exponentials and their sum in position order, the value
// accumulation o += p * v in position order, y = (x * inv) * w) is shared.

namespace {

// theta^(-2i / head_dim) for each rotated pair i, in double (kernels_ref.cpp:11-21).
std::vector<double> inverse_frequencies(int head_dim, float theta) {
  std::vector<double> f(static_cast<size_t>(head_dim / 2));
  for (size_t i = 0; i < f.size(); ++i) f[i] = std::pow(static_cast<double>(theta), -2.0 * static_cast<int>(i) / head_dim);
  return f;
}

}  // namespace

RopeTable::RopeTable(int head_dim, int max_pos_, float theta) : half(head_dim / 2), max_pos(max_pos_) {
  const std::vector<double> freq = inverse_frequencies(head_dim, theta);
  const size_t n = static_cast<size_t>(max_pos) * half;
  cos.assign(n, 0.f);
  sin.assign(n, 0.f);
  size_t at = 0;
  for (int p = 0; p < max_pos; ++p)
    for (double f : freq) {
      const double angle = p * f;
      cos[at] = static_cast<float>(std::cos(angle));
      sin[at] = static_cast<float>(std::sin(angle));
      ++at;
    }
}

namespace host {
namespace {

float sum_products_serial(const float* a, const float* b, int64_t n) {
  float acc = 0.f;
  for (int64_t i = 0; i < n; ++i) acc += a[i] * b[i];
  return acc;
}

float sum_products_four(const float* a, const float* b, int64_t n) {
  float part[4] = {0.f, 0.f, 0.f, 0.f};
  const int64_t whole = n - n % 4;
  for (int64_t base = 0; base < whole; base += 4)
    for (int lane = 0; lane < 4; ++lane) part[lane] += a[base + lane] * b[base + lane];
  for (int64_t i = whole; i < n; ++i) part[0] += a[i] * b[i];
  return (part[0] + part[1]) + (part[2] + part[3]);
}

inline float sum_products(Flavor f, const float* a, const float* b, int64_t n) {
  return f == Flavor::Cpu ? sum_products_four(a, b, n) : sum_products_serial(a, b, n);
}

// The RoPE angles of one position: pair i of a head vector, (lo, hi) = (x[i], x[i + half]), becomes
// (lo·c − hi·s, hi·c + lo·s), each product rounded on its own. src may equal dst.
struct Rotation {
  const float* c;
  const float* s;
  int half;
  void apply(const float* src, float* dst) const {
    for (int i = 0; i < half; ++i) {
      const float lo = src[i], hi = src[i + half];
      const float lo_c = lo * c[i], hi_s = hi * s[i], hi_c = hi * c[i], lo_s = lo * s[i];
      dst[i] = lo_c - hi_s;
      dst[i + half] = hi_c + lo_s;
    }
  }
};

Rotation rotation_at(const RopeTable& rt, int pos) {
  const size_t at = static_cast<size_t>(pos) * rt.half;
  return Rotation{rt.cos.data() + at, rt.sin.data() + at, rt.half};
}

// One layer's KV cache seen as rows of head_dim floats: [kv head][position][head_dim].
struct CacheRows {
  const KVLayer& kv;
  int head_dim;
  float* key(int kv_head, int pos) const { return kv.k + (static_cast<int64_t>(kv_head) * kv.max_ctx + pos) * head_dim; }
  float* value(int kv_head, int pos) const { return kv.v + (static_cast<int64_t>(kv_head) * kv.max_ctx + pos) * head_dim; }
};

// The step's keys (rotated when RoPE is fused) and values go into the cache at positions pos0 .. pos0+T-1
// before any query of the step reads it.
void store_step(const AttnArgs& a, const CacheRows& cache) {
  const int64_t width = static_cast<int64_t>(a.n_kv) * a.head_dim;
  for (int t = 0; t < a.T; ++t) {
    const int pos = a.pos0 + t;
    for (int g = 0; g < a.n_kv; ++g) {
      const int64_t from = t * width + static_cast<int64_t>(g) * a.head_dim;
      if (a.rope) rotation_at(*a.rope, pos).apply(a.k + from, cache.key(g, pos));
      else std::copy_n(a.k + from, a.head_dim, cache.key(g, pos));
      std::copy_n(a.v + from, a.head_dim, cache.value(g, pos));
    }
  }
}

// Output row of query token t, head h: softmax over positions 0..pos0+t of q·k / sqrt(head_dim), then
// the weighted sum of the value rows. `work` holds head_dim + (pos0 + T) floats.
void attend(const AttnArgs& a, const CacheRows& cache, Flavor f, int t, int h, float* work) {
  const int hd = a.head_dim, pos = a.pos0 + t, visible = pos + 1, group = h / (a.n_heads / a.n_kv);
  const int64_t row = (static_cast<int64_t>(t) * a.n_heads + h) * hd;
  const float* q = a.q + row;
  float* rotated = work;
  float* weight = work + hd;
  if (a.rope) {
    rotation_at(*a.rope, pos).apply(q, rotated);
    q = rotated;
  }
  const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
  float peak = -INFINITY;
  for (int j = 0; j < visible; ++j) {
    weight[j] = sum_products(f, q, cache.key(group, j), hd) * scale;
    peak = std::max(peak, weight[j]);
  }
  float total = 0.f;
  for (int j = 0; j < visible; ++j) {
    weight[j] = std::exp(weight[j] - peak);
    total += weight[j];
  }
  const float inv_total = 1.0f / total;
  float* out = a.out + row;
  std::fill_n(out, hd, 0.f);
  for (int j = 0; j < visible; ++j) {
    const float p = f == Flavor::Cpu ? weight[j] * inv_total : weight[j] / total;
    const float* v = cache.value(group, j);
    for (int i = 0; i < hd; ++i) out[i] += p * v[i];
  }
}

}  // namespace

void embed(const int32_t* tokens, int T, const Tensor& table, float* y) {
  for (int t = 0; t < T; ++t) {
    const int32_t id = tokens[t];
    EDGELM_CHECK(id >= 0 && id < table.rows, "token id out of range");
    dequantize_row(table, id, y + static_cast<int64_t>(t) * table.cols);
  }
}

void rmsnorm(const float* x, const float* w, float* y, int rows, int dim, float eps, Flavor f, ThreadPool* pool) {
  auto normalize = [&](int64_t first, int64_t last) {
    for (int64_t r = first; r < last; ++r) {
      const float* in = x + r * dim;
      float* out = y + r * dim;
      const float squares = sum_products(f, in, in, dim);
      const float inv = 1.0f / std::sqrt(squares / dim + eps);
      for (int i = 0; i < dim; ++i) out[i] = in[i] * inv * w[i];
    }
  };
  if (pool && f == Flavor::Cpu && rows > 8) pool->parallel_for(rows, normalize);
  else normalize(0, rows);
}

void rope(const float* x, float* y, int T, int n_heads, int hd, int pos0, const RopeTable& rt) {
  for (int t = 0; t < T; ++t) {
    EDGELM_CHECK(pos0 + t < rt.max_pos, "position beyond rope table");
    const Rotation r = rotation_at(rt, pos0 + t);
    for (int h = 0; h < n_heads; ++h) {
      const int64_t at = (static_cast<int64_t>(t) * n_heads + h) * hd;
      r.apply(x + at, y + at);
    }
  }
}

void attention(const AttnArgs& a, Flavor f, ThreadPool* pool) {
  EDGELM_CHECK(a.pos0 + a.T <= a.cache.max_ctx, "context overflow");
  if (a.rope && f == Flavor::Reference)  // the reference backend rotates through its rope op
    EDGELM_CHECK(a.pos0 + a.T <= a.rope->max_pos, "position beyond rope table");
  const CacheRows cache{a.cache, a.head_dim};
  store_step(a, cache);
  const size_t work = static_cast<size_t>(a.head_dim) + static_cast<size_t>(a.pos0 + a.T);
  auto items = [&](int64_t first, int64_t last) {
    std::vector<float> scratch(work);
    for (int64_t i = first; i < last; ++i)
      attend(a, cache, f, static_cast<int>(i / a.n_heads), static_cast<int>(i % a.n_heads), scratch.data());
  };
  const int64_t n = static_cast<int64_t>(a.T) * a.n_heads;
  if (pool && f == Flavor::Cpu) pool->parallel_for(n, items);
  else items(0, n);
}

void add(const float* a, const float* b, float* y, int64_t n) {
  std::transform(a, a + n, b, y, [](float u, float v) { return u + v; });
}
void mul(const float* a, const float* b, float* y, int64_t n) {
  std::transform(a, a + n, b, y, [](float u, float v) { return u * v; });
}
void silu(const float* x, float* y, int64_t n) {
  std::transform(x, x + n, y, [](float v) { return v / (1.0f + std::exp(-v)); });
}

}  // namespace host
}  // namespace edgelm

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

RopeTable::RopeTable(int head_dim, int max_pos_, float theta) : half(head_dim / 2), max_pos(max_pos_) {
  cos.resize(static_cast<size_t>(max_pos) * half);
  sin.resize(cos.size());
  for (int p = 0; p < max_pos; ++p)
    for (int i = 0; i < half; ++i) {
      const double ang = p * std::pow(static_cast<double>(theta), -2.0 * i / head_dim);  // in double
      cos[static_cast<size_t>(p) * half + i] = static_cast<float>(std::cos(ang));
      sin[static_cast<size_t>(p) * half + i] = static_cast<float>(std::sin(ang));
    }
}

namespace host {

float dot_f32(const float* a, const float* b, int64_t k) {
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

void embed(const int32_t* tokens, int T, const Tensor& table, float* y) {
  for (int t = 0; t < T; ++t) {
    EDGELM_CHECK(tokens[t] >= 0 && tokens[t] < table.rows, "token id out of range");
    dequantize_row(table, tokens[t], y + static_cast<int64_t>(t) * table.cols);
  }
}

void rmsnorm_ref(const float* x, const float* w, float* y, int rows, int dim, float eps) {
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + static_cast<int64_t>(r) * dim;
    float ss = 0.f;
    for (int i = 0; i < dim; ++i) ss += xr[i] * xr[i];
    const float inv = 1.0f / std::sqrt(ss / dim + eps);
    for (int i = 0; i < dim; ++i) y[static_cast<int64_t>(r) * dim + i] = xr[i] * inv * w[i];
  }
}

void rmsnorm(const float* x, const float* w, float* y, int rows, int dim, float eps, ThreadPool* pool) {
  auto body = [&](int64_t b, int64_t e) {
    for (int64_t r = b; r < e; ++r) {
      const float* xr = x + r * dim;
      float* yr = y + r * dim;
      const float inv = 1.0f / std::sqrt(dot_f32(xr, xr, dim) / dim + eps);
      for (int i = 0; i < dim; ++i) yr[i] = xr[i] * inv * w[i];
    }
  };
  if (pool && rows > 8) pool->parallel_for(rows, body);
  else body(0, rows);
}

void rope(const float* x, float* y, int T, int n_heads, int hd, int pos0, const RopeTable& rt) {
  const int h2 = hd / 2;
  for (int t = 0; t < T; ++t) {
    EDGELM_CHECK(pos0 + t < rt.max_pos, "position beyond rope table");
    const float* c = &rt.cos[static_cast<size_t>(pos0 + t) * h2];
    const float* s = &rt.sin[static_cast<size_t>(pos0 + t) * h2];
    for (int h = 0; h < n_heads; ++h) {
      const float* xi = x + (static_cast<int64_t>(t) * n_heads + h) * hd;
      float* yo = y + (static_cast<int64_t>(t) * n_heads + h) * hd;
      for (int i = 0; i < h2; ++i) {
        const float a = xi[i], b = xi[i + h2];
        yo[i] = a * c[i] - b * s[i];
        yo[i + h2] = b * c[i] + a * s[i];
      }
    }
  }
}

namespace {
// Appends this step's keys (rotated when the rope is fused) and values to the cache.
void append_kv(const AttnArgs& a) {
  const int hd = a.head_dim, h2 = hd / 2, kvd = a.n_kv * hd;
  const int64_t mc = a.cache.max_ctx;
  for (int t = 0; t < a.T; ++t) {
    const int pos = a.pos0 + t;
    for (int h = 0; h < a.n_kv; ++h) {
      const float* ks = a.k + static_cast<int64_t>(t) * kvd + h * hd;
      float* kd = a.cache.k + (h * mc + pos) * hd;
      if (a.rope) {
        const float* c = &a.rope->cos[static_cast<size_t>(pos) * h2];
        const float* s = &a.rope->sin[static_cast<size_t>(pos) * h2];
        for (int i = 0; i < h2; ++i) {
          kd[i] = ks[i] * c[i] - ks[i + h2] * s[i];
          kd[i + h2] = ks[i + h2] * c[i] + ks[i] * s[i];
        }
      } else {
        std::memcpy(kd, ks, sizeof(float) * hd);
      }
      std::memcpy(a.cache.v + (h * mc + pos) * hd, a.v + static_cast<int64_t>(t) * kvd + h * hd, sizeof(float) * hd);
    }
  }
}
}  // namespace

// edgelm's cpu attention (kernels_cpu.cpp:417-488, scalar path): one item per (token, head).
void attention(const AttnArgs& a, ThreadPool* pool) {
  const int hd = a.head_dim, h2 = hd / 2, qd = a.n_heads * hd, grp = a.n_heads / a.n_kv;
  const int64_t mc = a.cache.max_ctx;
  EDGELM_CHECK(a.pos0 + a.T <= mc, "context overflow");
  append_kv(a);
  const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
  auto body = [&](int64_t b, int64_t e) {
    std::vector<float> qbuf(static_cast<size_t>(hd)), sc(static_cast<size_t>(a.pos0 + a.T));
    for (int64_t idx = b; idx < e; ++idx) {
      const int t = static_cast<int>(idx / a.n_heads), h = static_cast<int>(idx % a.n_heads);
      const int pos = a.pos0 + t;
      const float* q = a.q + static_cast<int64_t>(t) * qd + h * hd;
      if (a.rope) {
        const float* c = &a.rope->cos[static_cast<size_t>(pos) * h2];
        const float* s = &a.rope->sin[static_cast<size_t>(pos) * h2];
        for (int i = 0; i < h2; ++i) {
          qbuf[i] = q[i] * c[i] - q[i + h2] * s[i];
          qbuf[i + h2] = q[i + h2] * c[i] + q[i] * s[i];
        }
        q = qbuf.data();
      }
      const float* kc = a.cache.k + (h / grp) * mc * hd;
      const float* vc = a.cache.v + (h / grp) * mc * hd;
      const int n = pos + 1;
      float mx = -INFINITY;
      for (int j = 0; j < n; ++j) {
        sc[j] = dot_f32(q, kc + static_cast<int64_t>(j) * hd, hd) * scale;
        mx = std::max(mx, sc[j]);
      }
      float sum = 0.f;
      for (int j = 0; j < n; ++j) sum += (sc[j] = std::exp(sc[j] - mx));
      const float inv = 1.0f / sum;
      float* o = a.out + static_cast<int64_t>(t) * qd + h * hd;
      std::fill(o, o + hd, 0.f);
      for (int j = 0; j < n; ++j) {
        const float p = sc[j] * inv;
        const float* vj = vc + static_cast<int64_t>(j) * hd;
        for (int i = 0; i < hd; ++i) o[i] += p * vj[i];
      }
    }
  };
  const int64_t items = static_cast<int64_t>(a.T) * a.n_heads;
  if (pool) pool->parallel_for(items, body);
  else body(0, items);
}

// edgelm's reference attention (kernels_ref.cpp:100-141).
void attention_ref(const AttnArgs& a) {
  const int hd = a.head_dim, kvd = a.n_kv * hd, qd = a.n_heads * hd, grp = a.n_heads / a.n_kv;
  EDGELM_CHECK(a.pos0 + a.T <= a.cache.max_ctx, "context overflow");
  std::vector<float> kr(static_cast<size_t>(a.T) * kvd), qr(static_cast<size_t>(a.T) * qd);
  const float* k = a.k;
  const float* q = a.q;
  if (a.rope) {
    rope(a.k, kr.data(), a.T, a.n_kv, hd, a.pos0, *a.rope);
    rope(a.q, qr.data(), a.T, a.n_heads, hd, a.pos0, *a.rope);
    k = kr.data();
    q = qr.data();
  }
  for (int t = 0; t < a.T; ++t)
    for (int h = 0; h < a.n_kv; ++h)
      for (int i = 0; i < hd; ++i) {
        const size_t dst = (static_cast<size_t>(h) * a.cache.max_ctx + a.pos0 + t) * hd + i;
        a.cache.k[dst] = k[static_cast<size_t>(t) * kvd + h * hd + i];
        a.cache.v[dst] = a.v[static_cast<size_t>(t) * kvd + h * hd + i];
      }
  const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
  std::vector<float> sc(static_cast<size_t>(a.pos0 + a.T));
  for (int t = 0; t < a.T; ++t)
    for (int h = 0; h < a.n_heads; ++h) {
      const float* qv = q + static_cast<size_t>(t) * qd + h * hd;
      const float* kc = a.cache.k + static_cast<size_t>(h / grp) * a.cache.max_ctx * hd;
      const float* vc = a.cache.v + static_cast<size_t>(h / grp) * a.cache.max_ctx * hd;
      const int n = a.pos0 + t + 1;
      float mx = -INFINITY;
      for (int j = 0; j < n; ++j) {
        float d = 0.f;
        for (int i = 0; i < hd; ++i) d += qv[i] * kc[static_cast<size_t>(j) * hd + i];
        sc[j] = d * scale;
        mx = std::max(mx, sc[j]);
      }
      float sum = 0.f;
      for (int j = 0; j < n; ++j) sum += (sc[j] = std::exp(sc[j] - mx));
      float* o = a.out + static_cast<size_t>(t) * qd + h * hd;
      for (int i = 0; i < hd; ++i) o[i] = 0.f;
      for (int j = 0; j < n; ++j)
        for (int i = 0; i < hd; ++i) o[i] += sc[j] / sum * vc[static_cast<size_t>(j) * hd + i];
    }
}

void add(const float* a, const float* b, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = a[i] + b[i];
}
void silu(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = x[i] / (1.0f + std::exp(-x[i]));
}
void mul(const float* a, const float* b, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = a[i] * b[i];
}

}  // namespace host
}  // namespace edgelm

// Host-side pieces around the hot path: a thread pool and the non-matmul ops (embedding, RMSNorm,
// RoPE, causal GQA attention over the KV cache, elementwise ops). They reproduce edgelm's cpu and
// reference backends' arithmetic on the x86 scalar path (kernels_cpu.cpp:32-43, 326-337, 413-492;
// kernels_ref.cpp:11-21, 41-151), so a session mixing them with the hip backend computes what
// edgelm's own session computes.
#pragma once
#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include "edgelm/backend.hpp"

namespace edgelm {

// Fixed-size pool: each parallel_for hands worker i the i-th of `size()` contiguous slices of
// [0, n) (results never depend on the thread count: every item is computed independently).
// Workers spin briefly on their epoch counter, then park on a condition variable.
class ThreadPool {
 public:
  explicit ThreadPool(int threads);
  ~ThreadPool();
  ThreadPool(const ThreadPool&) = delete;
  ThreadPool& operator=(const ThreadPool&) = delete;
  int size() const { return n_; }
  void parallel_for(int64_t n, const std::function<void(int64_t, int64_t)>& fn);

 private:
  struct alignas(64) Slot {
    std::atomic<uint64_t> epoch{0};
    std::atomic<uint64_t> done{0};
  };
  void worker(int id);
  int n_;
  std::vector<std::thread> threads_;
  std::vector<Slot> slots_;
  uint64_t epoch_ = 0;
  const std::function<void(int64_t, int64_t)>* fn_ = nullptr;
  int64_t items_ = 0;
  std::atomic<bool> stop_{false};
  std::atomic<int> sleepers_{0};
  std::mutex mu_;
  std::condition_variable cv_;
};

struct AttnArgs {
  const float* q;  // [T, nh*hd]
  const float* k;  // [T, nkv*hd] new keys (before rope when rope != nullptr)
  const float* v;  // [T, nkv*hd]
  float* out;      // [T, nh*hd]
  int T, pos0, n_heads, n_kv, head_dim;
  KVLayer cache;
  const RopeTable* rope;
};

namespace host {
// Which of edgelm's two host backends an op reproduces. They round alike except in how a dot product
// or sum of squares accumulates (one running sum, or four over the index mod 4) and in the softmax
// weight of a position (e / sum, or e * (1 / sum)).
enum class Flavor { Reference, Cpu };

void embed(const int32_t* tokens, int T, const Tensor& table, float* y);
// Reference runs serially; Cpu splits rows over `pool` (when non-null).
void rmsnorm(const float* x, const float* w, float* y, int rows, int dim, float eps, Flavor f, ThreadPool* pool);
void rope(const float* x, float* y, int T, int n_heads, int head_dim, int pos0, const RopeTable& rt);
// Appends the step's keys and values to the cache, then one output row per (token, head); Cpu splits
// the rows over `pool` (when non-null).
void attention(const AttnArgs& a, Flavor f, ThreadPool* pool);
void add(const float* a, const float* b, float* y, int64_t n);
void silu(const float* x, float* y, int64_t n);
void mul(const float* a, const float* b, float* y, int64_t n);
}  // namespace host

}  // namespace edgelm

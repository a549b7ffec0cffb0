// Session (reference runtime.cpp:8-91): fuse, instantiate backends, partition, plan the activation
// arena, allocate the KV cache, then run forward() over the partitions in op order.
#include "edgelm/runtime.hpp"

#include <algorithm>
#include <cstring>

#include "edgelm/host_ops.hpp"

namespace edgelm {

Session::Session(const Model& model, SessionOptions opt) : model_(model), opt_(std::move(opt)), graph_(model.graph) {
  const Config& c = model.cfg;
  EDGELM_CHECK(opt_.max_batch >= 1 && opt_.max_ctx >= 1, "bad session sizes");
  opt_.max_ctx = std::min(opt_.max_ctx, c.max_seq);
  opt_.max_batch = std::min(opt_.max_batch, opt_.max_ctx);
  if (opt_.fuse) optimize(graph_);

  for (const std::string& b : opt_.backends)
    if (b != "reference" && b != "ref") backends_.push_back(make_backend(b));
  backends_.push_back(make_reference_backend());
  std::vector<Backend*> pref;
  for (auto& b : backends_) pref.push_back(b.get());
  parts_ = partition_graph(graph_, pref);
  for (auto& b : backends_) b->prepare(graph_, parts_);

  const int L = opt_.all_logits ? opt_.max_batch : 1;
  plan_ = plan_memory(graph_, opt_.max_batch, L);
  arena_.assign(plan_.arena_bytes + 64, 0);
  uint8_t* base = arena_.data() + (64 - reinterpret_cast<uintptr_t>(arena_.data()) % 64) % 64;
  ctx_.graph = &graph_;
  ctx_.ptr.assign(graph_.tensors.size(), nullptr);
  for (size_t t = 0; t < graph_.tensors.size(); ++t)
    if (plan_.offset[t] >= 0) ctx_.ptr[t] = reinterpret_cast<float*>(base + plan_.offset[t]);

  const size_t per_layer = static_cast<size_t>(c.n_kv_heads) * opt_.max_ctx * c.head_dim;
  kcache_.assign(per_layer * c.n_layers, 0.f);
  vcache_.assign(per_layer * c.n_layers, 0.f);
  for (int l = 0; l < c.n_layers; ++l)
    ctx_.kv.push_back({kcache_.data() + l * per_layer, vcache_.data() + l * per_layer, opt_.max_ctx});
  rope_ = RopeTable(c.head_dim, opt_.max_ctx, c.rope_theta);
  ctx_.rope = &rope_;
  pool_ = std::make_unique<ThreadPool>(opt_.threads);
  ctx_.pool = pool_.get();
  ctx_.act_quant = opt_.act_quant;
}

Session::~Session() = default;

const float* Session::forward(const int32_t* tokens, int n) {
  EDGELM_CHECK(n >= 1 && n <= opt_.max_batch, "forward: n must be in [1, max_batch]");
  EDGELM_CHECK(pos_ + n <= opt_.max_ctx, "forward: context full");
  ctx_.T = n;
  ctx_.L = opt_.all_logits ? n : 1;
  ctx_.pos0 = pos_;
  std::memcpy(ctx_.ptr[graph_.input], tokens, sizeof(int32_t) * static_cast<size_t>(n));
  for (const Partition& p : parts_)
    if (!p.backend->run_partition(p, ctx_))
      for (int i = p.begin; i < p.end; ++i) p.backend->run(graph_.ops[i], ctx_);
  pos_ += n;
  return ctx_.ptr[graph_.output];
}

const float* Session::prefill(const std::vector<int32_t>& tokens) {
  EDGELM_CHECK(!tokens.empty(), "prefill: empty prompt");
  const float* out = nullptr;
  for (size_t i = 0; i < tokens.size(); i += static_cast<size_t>(opt_.max_batch)) {
    const int n = static_cast<int>(std::min<size_t>(static_cast<size_t>(opt_.max_batch), tokens.size() - i));
    out = forward(tokens.data() + i, n);
  }
  return out;
}

int32_t argmax(const float* logits, int n) {
  return static_cast<int32_t>(std::max_element(logits, logits + n) - logits);
}

}  // namespace edgelm

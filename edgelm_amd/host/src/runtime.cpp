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
  for (const Partition& p : parts_)
    for (int i = p.begin; i < p.end; ++i)
      for (int t : graph_.ops[i].out)
        if (t == graph_.output) output_backend_ = p.backend;

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

int32_t Session::greedy(const int32_t* tokens, int n) {
  Backend* b = output_backend_;
  const bool on_dev = b && b->keep_output(true);
  const float* lg = nullptr;
  int32_t tok = 0;
  try {
    lg = forward(tokens, n);
    if (on_dev && !b->argmax_output(ctx_, &tok)) EDGELM_CHECK(false, "greedy: the output's backend lost its logits");
  } catch (...) {
    if (b) b->keep_output(false);
    throw;
  }
  if (b) b->keep_output(false);
  if (!on_dev) tok = argmax(lg + static_cast<size_t>(ctx_.L - 1) * static_cast<size_t>(vocab()), vocab());
  return tok;
}

int32_t Session::greedy_prefill(const std::vector<int32_t>& tokens) {
  EDGELM_CHECK(!tokens.empty(), "prefill: empty prompt");
  const size_t mb = static_cast<size_t>(opt_.max_batch);
  const size_t last = (tokens.size() - 1) / mb * mb;  // start of the final chunk
  if (last) prefill(std::vector<int32_t>(tokens.begin(), tokens.begin() + static_cast<std::ptrdiff_t>(last)));
  return greedy(tokens.data() + last, static_cast<int>(tokens.size() - last));
}

int32_t argmax(const float* logits, int n) {
  return static_cast<int32_t>(std::max_element(logits, logits + n) - logits);
}

}  // namespace edgelm

// Session: one model instance ready to run (edgelm's Session interface, runtime.hpp:17-67). Building
// one fuses the graph (unless asked not to), instantiates the backends in preference order with the
// reference backend last, partitions the graph, lets each backend prepare for its partitions, plans
// the host activation arena and allocates the KV cache and the RoPE table; forward() then runs T tokens
// through the partitions in op order.
#include <algorithm>
#include <cstring>
#include <stdexcept>

#include "edgelm/host_ops.hpp"
#include "edgelm/runtime.hpp"

namespace edgelm {
namespace {

SessionOptions fit_to_model(SessionOptions o, const Config& c) {
  if (o.max_batch < 1 || o.max_ctx < 1) throw std::runtime_error("edgelm: a session needs max_batch >= 1 and max_ctx >= 1");
  o.max_ctx = std::min(o.max_ctx, c.max_seq);      // no position past what the model was made for
  o.max_batch = std::min(o.max_batch, o.max_ctx);  // and no chunk longer than the context
  return o;
}

}  // namespace

Session::Session(const Model& model, SessionOptions opt)
    : model_(model), opt_(fit_to_model(std::move(opt), model.cfg)), graph_(model.graph) {
  if (opt_.fuse) optimize(graph_);

  for (const std::string& name : opt_.backends)
    if (name != "reference" && name != "ref") backends_.push_back(make_backend(name));
  backends_.push_back(make_reference_backend());
  std::vector<Backend*> order(backends_.size());
  std::transform(backends_.begin(), backends_.end(), order.begin(), [](const std::unique_ptr<Backend>& b) { return b.get(); });
  parts_ = partition_graph(graph_, order);
  for (Backend* b : order) b->prepare(graph_, parts_);
  for (const Partition& p : parts_)
    for (int i = p.begin; i < p.end; ++i)
      if (std::count(graph_.ops[i].out.begin(), graph_.ops[i].out.end(), graph_.output)) output_backend_ = p.backend;

  // host activations: one 64-byte aligned arena laid out by the planner for max_batch tokens
  plan_ = plan_memory(graph_, opt_.max_batch, opt_.all_logits ? opt_.max_batch : 1);
  arena_.assign(plan_.arena_bytes + 64, 0);
  uint8_t* base = arena_.data() + (64 - reinterpret_cast<uintptr_t>(arena_.data()) % 64) % 64;
  ctx_.graph = &graph_;
  ctx_.ptr.assign(graph_.tensors.size(), nullptr);
  for (size_t t = 0; t < graph_.tensors.size(); ++t)
    if (plan_.offset[t] >= 0) ctx_.ptr[t] = reinterpret_cast<float*>(base + plan_.offset[t]);

  // KV cache: per layer a [n_kv][max_ctx][head_dim] block of keys, then one of values
  const Config& c = model_.cfg;
  const size_t block = static_cast<size_t>(c.n_kv_heads) * static_cast<size_t>(opt_.max_ctx) * static_cast<size_t>(c.head_dim);
  kv_.assign(2 * block * static_cast<size_t>(c.n_layers), 0.f);
  for (int l = 0; l < c.n_layers; ++l) {
    float* k = kv_.data() + 2 * block * static_cast<size_t>(l);
    ctx_.kv.push_back(KVLayer{k, k + block, opt_.max_ctx});
  }
  rope_ = RopeTable(c.head_dim, opt_.max_ctx, c.rope_theta);
  ctx_.rope = &rope_;
  pool_ = std::make_unique<ThreadPool>(opt_.threads);
  ctx_.pool = pool_.get();
  ctx_.act_quant = opt_.act_quant;
}

Session::~Session() = default;

const float* Session::forward(const int32_t* tokens, int n) {
  if (n < 1 || n > opt_.max_batch) throw std::runtime_error("edgelm: forward takes 1 .. max_batch tokens");
  if (pos_ + n > opt_.max_ctx) throw std::runtime_error("edgelm: the context is full");
  ctx_.T = n;
  ctx_.L = opt_.all_logits ? n : 1;
  ctx_.pos0 = pos_;
  std::memcpy(ctx_.ptr[graph_.input], tokens, sizeof(int32_t) * static_cast<size_t>(n));
  for (const Partition& p : parts_) {
    if (p.backend->run_partition(p, ctx_)) continue;  // the backend ran the whole partition itself
    for (int i = p.begin; i < p.end; ++i) p.backend->run(graph_.ops[i], ctx_);
  }
  pos_ += n;
  return ctx_.ptr[graph_.output];
}

const float* Session::prefill(const std::vector<int32_t>& tokens) {
  if (tokens.empty()) throw std::runtime_error("edgelm: prefill of an empty prompt");
  const float* logits = nullptr;
  for (size_t at = 0; at < tokens.size();) {
    const int n = static_cast<int>(std::min(tokens.size() - at, static_cast<size_t>(opt_.max_batch)));
    logits = forward(tokens.data() + at, n);
    at += static_cast<size_t>(n);
  }
  return logits;
}

int32_t Session::greedy(const int32_t* tokens, int n) {
  Backend* b = output_backend_;
  const bool on_device = b && b->keep_output(true);
  struct Release {  // the output goes back to the host arena however the forward ends
    Backend* b;
    ~Release() {
      if (b) b->keep_output(false);
    }
  } release{b};
  const float* logits = forward(tokens, n);
  int32_t next = 0;
  if (on_device) {
    if (!b->argmax_output(ctx_, &next)) throw std::runtime_error("edgelm: greedy: the output's backend lost its logits");
    return next;
  }
  const int64_t vocab = model_.cfg.vocab;
  return argmax(logits + static_cast<size_t>(ctx_.L - 1) * static_cast<size_t>(vocab), static_cast<int>(vocab));
}

int32_t Session::greedy_steps(int32_t first, int n, int32_t* tokens) {
  if (n < 1) throw std::runtime_error("edgelm: greedy_steps takes n >= 1");
  if (pos_ + n > opt_.max_ctx) throw std::runtime_error("edgelm: the context is full");
  std::vector<int32_t> own;
  if (!tokens) own.resize(static_cast<size_t>(n));
  int32_t* out = tokens ? tokens : own.data();
  Backend* b = output_backend_;
  if (parts_.size() == 1 && parts_[0].backend == b && b->keep_output(true)) {
    struct Release {
      Backend* b;
      ~Release() { b->keep_output(false); }
    } release{b};
    ctx_.T = 1;
    ctx_.L = 1;
    ctx_.pos0 = pos_;
    if (b->greedy_steps(parts_[0], ctx_, first, n, out)) {
      pos_ += n;
      return out[n - 1];
    }
  }
  int32_t tok = first;
  for (int i = 0; i < n; ++i) out[i] = tok = greedy(&tok, 1);
  return tok;
}

int32_t Session::greedy_prefill(const std::vector<int32_t>& tokens) {
  if (tokens.empty()) throw std::runtime_error("edgelm: prefill of an empty prompt");
  const size_t chunk = static_cast<size_t>(opt_.max_batch), tail = (tokens.size() - 1) / chunk * chunk;
  if (tail) prefill(std::vector<int32_t>(tokens.begin(), tokens.begin() + static_cast<std::ptrdiff_t>(tail)));
  return greedy(tokens.data() + tail, static_cast<int>(tokens.size() - tail));
}

// edgelm's argmax (tokenizer.cpp:187-189): std::max_element's first largest element
int32_t argmax(const float* logits, int n) { return static_cast<int32_t>(std::max_element(logits, logits + n) - logits); }

}  // namespace edgelm

// The runtime around the delegate: graph rewrites, the activation arena planner and the Session
// (edgelm's interfaces: passes.hpp:12-38, runtime.hpp:17-67). The MATMUL family goes to the `hip`
// backend; the remaining ops run on the host ("cpu" / "reference" backends of this build, which carry
// no quantized-matmul code at all).
#pragma once
#include <memory>
#include <string>
#include <vector>

#include "edgelm/backend.hpp"
#include "edgelm/model.hpp"

namespace edgelm {

// Fusion rewrites (edgelm's passes.hpp:12-38); each returns how many fused ops it made.
int fuse_swiglu(Graph& g);
int fuse_shared_input(Graph& g);
int fuse_residual(Graph& g);
int fuse_rope_attention(Graph& g);
struct FusionStats {
  int swiglu = 0, shared_input = 0, residual = 0, rope = 0;
  size_t ops_before = 0, ops_after = 0;
};
FusionStats optimize(Graph& g);

struct MemoryPlan {
  std::vector<int64_t> offset, bytes;
  std::vector<int> first, last;
  size_t arena_bytes = 0, naive_bytes = 0;
  int n_planned = 0;
};
MemoryPlan plan_memory(const Graph& g, int T, int L);
bool plan_is_valid(const MemoryPlan& p);

struct SessionOptions {
  std::vector<std::string> backends{"hip", "cpu"};  // preference order; reference is appended last
  int threads = 1;
  int max_ctx = 1024;
  int max_batch = 128;
  bool all_logits = false;
  bool fuse = true;
  bool act_quant = false;
};

class Session {
 public:
  Session(const Model& model, SessionOptions opt);
  ~Session();
  Session(const Session&) = delete;
  Session& operator=(const Session&) = delete;

  const float* forward(const int32_t* tokens, int n);
  const float* prefill(const std::vector<int32_t>& tokens);
  const float* decode(int32_t token) { return forward(&token, 1); }
  // Greedy next token after forward(tokens, n) / prefill(tokens): the argmax of the last row of
  // logits, taken on the device by the output's backend when it offers argmax_output (the logits
  // then stay there), else on the host arena's copy as edgelm's bench does (main.cpp:199-213).
  int32_t greedy(const int32_t* tokens, int n);
  int32_t greedy_prefill(const std::vector<int32_t>& tokens);
  // n greedy decode steps, the first from token `first`, each later one from the token the step
  // before chose: the same tokens as n calls of greedy(&tok, 1). A backend that runs the whole graph
  // and keeps the logits may queue the steps back to back (greedy_steps hook); tokens (may be null)
  // gets all n, and the last one is returned.
  int32_t greedy_steps(int32_t first, int n, int32_t* tokens);
  void reset() { pos_ = 0; }
  int pos() const { return pos_; }

  const Graph& graph() const { return graph_; }
  const std::vector<Partition>& partitions() const { return parts_; }
  const MemoryPlan& plan() const { return plan_; }
  const SessionOptions& options() const { return opt_; }
  int vocab() const { return model_.cfg.vocab; }

 private:
  const Model& model_;
  SessionOptions opt_;
  Graph graph_;
  MemoryPlan plan_;
  std::vector<std::unique_ptr<Backend>> backends_;
  std::vector<Partition> parts_;
  std::unique_ptr<ThreadPool> pool_;
  std::vector<uint8_t> arena_;
  std::vector<float> kv_;  // per layer: keys [n_kv][max_ctx][head_dim], then values
  RopeTable rope_;
  ExecContext ctx_;
  int pos_ = 0;
  Backend* output_backend_ = nullptr;  // backend of the op writing the graph output
};

int32_t argmax(const float* logits, int n);

}  // namespace edgelm

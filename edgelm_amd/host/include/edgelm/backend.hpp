// Delegate interface (reference include/edgelm/backend.hpp:15-51): a backend declares the ops it
// supports; the partitioner gives each op to the first backend in preference order that claims it
// and groups consecutive ops into partitions. The names, members and semantics are edgelm's, so the
// `hip` backend of this build plugs into edgelm's Session unchanged.
#pragma once
#include <memory>
#include <string>
#include <vector>

#include "edgelm/graph.hpp"

namespace edgelm {

class ThreadPool;

struct RopeTable {
  int half = 0, max_pos = 0;
  std::vector<float> cos, sin;  // [pos][half]
  RopeTable() = default;
  RopeTable(int head_dim, int max_pos, float theta);
};

struct KVLayer {  // one layer's cache, [kv_head][pos][head_dim]
  float* k = nullptr;
  float* v = nullptr;
  int max_ctx = 0;
};

constexpr int kActBlock = 32;
struct ActBuf {
  int8_t* q = nullptr;  // [T, K]
  float* d = nullptr;   // [T, K/32]
};

struct ExecContext {
  const Graph* graph = nullptr;
  std::vector<float*> ptr;  // activation tensor -> host arena address
  int T = 0, L = 0, pos0 = 0;
  std::vector<KVLayer> kv;
  const RopeTable* rope = nullptr;
  ThreadPool* pool = nullptr;
  std::vector<float*> scratch;
  bool act_quant = false;  // int8 activations for q8/q4 matmuls
  ActBuf aq;               // host scratch the cpu matmuls use; the hip backend ignores it
  const Tensor& tensor(int i) const { return graph->tensors[i]; }
  float* f(int i) const { return ptr[i]; }
  int64_t rows(int i) const;
};

struct Partition;

class Backend {
 public:
  virtual ~Backend() = default;
  virtual const char* name() const = 0;
  virtual bool supports(const Graph& g, const Op& op) const = 0;
  virtual void run(const Op& op, ExecContext& ctx) = 0;
  // Optional (default: nothing), called once by the Session after partitioning: lets a device
  // backend keep activations on its device between its own consecutive ops and copy to the host
  // arena only what other backends read. Source-compatible with edgelm's Backend.
  virtual void prepare(const Graph&, const std::vector<Partition>&) {}
  // Optional (default: false = not handled): run the whole partition at once (a device backend may
  // replay it as a captured graph). Returning true means every op of the partition ran and the
  // host arena holds what other backends read, as after run().
  virtual bool run_partition(const Partition&, ExecContext&) { return false; }
  // Optional (default: false = not handled), for greedy sampling: true means this backend produces
  // the graph output and, until called again with true, leaves it where it computes it instead of
  // copying it into the host arena; argmax_output() then answers for each forward.
  virtual bool keep_output(bool) { return false; }
  // Optional: the argmax (edgelm's argmax, tokenizer.cpp:187-189) of the graph output's last row,
  // taken where the output lives; false if this backend cannot.
  virtual bool argmax_output(const ExecContext&, int32_t*) { return false; }
  // Optional (default: false = not handled), for greedy decoding when this backend runs the whole
  // graph as one partition and keeps its output: n decode steps at positions ctx.pos0 .. + n - 1,
  // the first from token `first` and each later one from the argmax of the step before, fed back
  // where the logits are, so the steps can be queued back to back; out[i] is step i's argmax.
  virtual bool greedy_steps(const Partition&, ExecContext&, int32_t /*first*/, int /*n*/, int32_t* /*out*/) {
    return false;
  }
};

std::unique_ptr<Backend> make_reference_backend();
std::unique_ptr<Backend> make_cpu_backend();
// The MI355X delegate ("hip"): MATMUL / MATMUL_N / MATMUL_ADD / FFN_SWIGLU with q8 or q4 weights,
// EMBED (q8/q4 table), RMSNORM, ATTENTION and LAST_ROWS, activations kept in HBM between its ops.
// Throws if no gfx950 device is usable.
std::unique_ptr<Backend> make_hip_backend(int device = 0);
// "hip-matmul": the matmul family only (the template of edgelm's MatmulOnlyBackend).
std::unique_ptr<Backend> make_hip_matmul_backend(int device = 0);
// Same claims as the hip (layer_ops) or hip-matmul backend but no device: for partition
// inspection only (run() throws).
std::unique_ptr<Backend> make_hip_planning_backend(bool layer_ops = true);
std::unique_ptr<Backend> make_backend(const std::string& name);

struct Partition {
  Backend* backend = nullptr;
  int begin = 0, end = 0;  // op range [begin, end)
};

std::vector<Partition> partition_graph(const Graph& g, const std::vector<Backend*>& preference);
std::string describe_partitions(const Graph& g, const std::vector<Partition>& parts);

}  // namespace edgelm

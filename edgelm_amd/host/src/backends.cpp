// The backends of this runtime besides the delegate, the registry that makes backends by name, and the
// partitioner (edgelm's contract: backend.hpp:30-51, backends.cpp:158-201).
//
// "reference" (always last in a session's preference list) and "cpu" are host backends for the ops
// around the hot path: EMBED, RMSNORM, ROPE, ATTENTION, LAST_ROWS and the elementwise ADD / SILU / MUL,
// with edgelm's arithmetic (host_ops.cpp). Neither claims MATMUL, MATMUL_N, MATMUL_ADD or FFN_SWIGLU:
// the quantized matmul family exists only in the `hip` delegate, so a session without a working GPU
// fails to partition ("no backend claims ...") instead of running matmuls on the CPU.
#include <algorithm>
#include <cstring>
#include <functional>
#include <map>
#include <sstream>
#include <stdexcept>

#include "edgelm/backend.hpp"
#include "edgelm/host_ops.hpp"

namespace edgelm {

int64_t ExecContext::rows(int i) const {
  switch (graph->tensors[i].rows_sym) {
    case RowSym::T: return T;
    case RowSym::L: return L;
    default: return graph->tensors[i].rows;
  }
}

namespace {

bool is_matmul_family(OpType t) {
  return t == OpType::MATMUL || t == OpType::MATMUL_N || t == OpType::MATMUL_ADD || t == OpType::FFN_SWIGLU;
}

// The operands of one ATTENTION op (iattr: layer, n_heads, n_kv, fused rope) in this step.
AttnArgs attention_operands(const Op& op, const ExecContext& c) {
  const int layer = op.iattr[0];
  if (layer < 0 || layer >= static_cast<int>(c.kv.size()))
    throw std::runtime_error("edgelm: attention names layer " + std::to_string(layer));
  AttnArgs a{c.f(op.in[0]), c.f(op.in[1]), c.f(op.in[2]), c.f(op.out[0]), static_cast<int>(c.rows(op.in[0])), c.pos0,
             op.iattr[1], op.iattr[2], 0, c.kv[layer], op.iattr[3] ? c.rope : nullptr};
  a.head_dim = static_cast<int>(c.tensor(op.in[0]).cols / a.n_heads);
  return a;
}

// The ops whose host arithmetic is the same in both host backends.
bool run_elementwise(const Op& op, ExecContext& c) {
  const int64_t n = c.rows(op.out[0]) * c.tensor(op.out[0]).cols;
  float* y = c.f(op.out[0]);
  switch (op.type) {
    case OpType::ADD: host::add(c.f(op.in[0]), c.f(op.in[1]), y, n); return true;
    case OpType::MUL: host::mul(c.f(op.in[0]), c.f(op.in[1]), y, n); return true;
    case OpType::SILU: host::silu(c.f(op.in[0]), y, n); return true;
    case OpType::ROPE:
      host::rope(c.f(op.in[0]), y, static_cast<int>(c.rows(op.in[0])), op.iattr[0], op.iattr[1], c.pos0, *c.rope);
      return true;
    default: return false;
  }
}

const float* norm_weight(const ExecContext& c, const Op& op) { return static_cast<const float*>(c.tensor(op.in[1]).data); }

[[noreturn]] void unhandled(const char* backend, const Op& op) {
  throw std::runtime_error(std::string("edgelm: the ") + backend + " backend cannot run " + op_name(op.type));
}

// edgelm's reference backend (serial) for everything but the matmul family.
class HostReference final : public Backend {
 public:
  const char* name() const override { return "reference"; }
  bool supports(const Graph&, const Op& op) const override { return !is_matmul_family(op.type); }
  void run(const Op& op, ExecContext& c) override {
    if (run_elementwise(op, c)) return;
    switch (op.type) {
      case OpType::EMBED:
        host::embed(reinterpret_cast<const int32_t*>(c.f(op.in[0])), c.T, c.tensor(op.in[1]), c.f(op.out[0]));
        break;
      case OpType::RMSNORM:
        host::rmsnorm(c.f(op.in[0]), norm_weight(c, op), c.f(op.out[0]), static_cast<int>(c.rows(op.in[0])),
                      static_cast<int>(c.tensor(op.in[0]).cols), op.fattr[0], host::Flavor::Reference, nullptr);
        break;
      case OpType::ATTENTION: host::attention(attention_operands(op, c), host::Flavor::Reference, nullptr); break;
      case OpType::LAST_ROWS: {
        const int64_t cols = c.tensor(op.in[0]).cols, keep = c.rows(op.out[0]), skip = c.rows(op.in[0]) - keep;
        if (skip < 0) throw std::runtime_error("edgelm: LAST_ROWS keeps more rows than it has");
        std::memmove(c.f(op.out[0]), c.f(op.in[0]) + skip * cols, sizeof(float) * static_cast<size_t>(keep * cols));
        break;
      }
      default: unhandled(name(), op);
    }
  }
};

// edgelm's cpu backend (threaded) for RMSNORM, ATTENTION and the elementwise ops; like edgelm's, it
// leaves EMBED and LAST_ROWS to the reference backend.
class HostCpu final : public Backend {
 public:
  const char* name() const override { return "cpu"; }
  bool supports(const Graph&, const Op& op) const override {
    return !is_matmul_family(op.type) && op.type != OpType::EMBED && op.type != OpType::LAST_ROWS;
  }
  void run(const Op& op, ExecContext& c) override {
    if (run_elementwise(op, c)) return;
    if (op.type == OpType::RMSNORM)
      host::rmsnorm(c.f(op.in[0]), norm_weight(c, op), c.f(op.out[0]), static_cast<int>(c.rows(op.in[0])),
                    static_cast<int>(c.tensor(op.in[0]).cols), op.fattr[0], host::Flavor::Cpu, c.pool);
    else if (op.type == OpType::ATTENTION)
      host::attention(attention_operands(op, c), host::Flavor::Cpu, c.pool);
    else
      unhandled(name(), op);
  }
};

using Factory = std::function<std::unique_ptr<Backend>()>;

const std::map<std::string, Factory>& registry() {
  static const std::map<std::string, Factory> table = {
      {"reference", [] { return make_reference_backend(); }},
      {"ref", [] { return make_reference_backend(); }},
      {"cpu", [] { return make_cpu_backend(); }},
      {"hip", [] { return make_hip_backend(0); }},
      {"hip-matmul", [] { return make_hip_matmul_backend(0); }},
  };
  return table;
}

}  // namespace

std::unique_ptr<Backend> make_reference_backend() { return std::make_unique<HostReference>(); }
std::unique_ptr<Backend> make_cpu_backend() { return std::make_unique<HostCpu>(); }

std::unique_ptr<Backend> make_backend(const std::string& name) {
  const auto& table = registry();
  const auto it = table.find(name);
  if (it == table.end()) throw std::runtime_error("edgelm: unknown backend " + name);
  return it->second();
}

// Each op goes to the first backend in `preference` that claims it; a partition is a maximal run of
// consecutive ops with the same backend.
std::vector<Partition> partition_graph(const Graph& g, const std::vector<Backend*>& preference) {
  std::vector<Partition> parts;
  const int n = static_cast<int>(g.ops.size());
  for (int i = 0; i < n; ++i) {
    const Op& op = g.ops[i];
    const auto who = std::find_if(preference.begin(), preference.end(), [&](Backend* b) { return b->supports(g, op); });
    if (who == preference.end()) throw std::runtime_error(std::string("edgelm: no backend claims ") + op_name(op.type));
    if (parts.empty() || parts.back().backend != *who) parts.push_back(Partition{*who, i, i});
    parts.back().end = i + 1;
  }
  return parts;
}

// "<partitions> partitions | <backend>: <ops> ops in <parts> | ..." (backends in order of first use),
// then one line per partition when there are at most eight.
std::string describe_partitions(const Graph& g, const std::vector<Partition>& parts) {
  std::vector<std::string> order;
  std::map<std::string, std::pair<int, int>> tally;  // backend -> (ops, partitions)
  for (const Partition& p : parts) {
    const std::string b = p.backend->name();
    if (!tally.count(b)) order.push_back(b);
    tally[b].first += p.end - p.begin;
    tally[b].second += 1;
  }
  std::ostringstream os;
  os << parts.size() << " partitions";
  for (const std::string& b : order) os << " | " << b << ": " << tally[b].first << " ops in " << tally[b].second;
  if (parts.size() <= 8)
    for (const Partition& p : parts)
      os << "\n  ops " << p.begin << ".." << p.end - 1 << " on " << p.backend->name() << " (" << op_name(g.ops[p.begin].type)
         << (p.end - p.begin > 1 ? std::string(" .. ") + op_name(g.ops[p.end - 1].type) : std::string()) << ")";
  return os.str();
}

}  // namespace edgelm

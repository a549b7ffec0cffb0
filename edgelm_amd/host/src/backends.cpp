// The host backends of this build and the partitioner (reference backends.cpp:36-201).
//
// "reference" (always appended last) and "cpu" run the non-matmul ops on the host. Neither carries
// an implementation of the quantized matmul family: MATMUL / MATMUL_N / MATMUL_ADD / FFN_SWIGLU
// exist only in the `hip` backend, so a session without a working GPU fails at partitioning
// ("no backend supports ...") instead of falling back to the CPU.
#include <cstring>
#include <map>
#include <sstream>

#include "edgelm/backend.hpp"
#include "edgelm/host_ops.hpp"

namespace edgelm {

int64_t ExecContext::rows(int i) const {
  const Tensor& t = graph->tensors[i];
  return t.rows_sym == RowSym::T ? T : t.rows_sym == RowSym::L ? L : t.rows;
}

namespace {

bool is_matmul_family(OpType t) {
  return t == OpType::MATMUL || t == OpType::MATMUL_N || t == OpType::MATMUL_ADD || t == OpType::FFN_SWIGLU;
}

AttnArgs attn_args(const Op& op, const ExecContext& c) {
  AttnArgs a{};
  a.q = c.f(op.in[0]);
  a.k = c.f(op.in[1]);
  a.v = c.f(op.in[2]);
  a.out = c.f(op.out[0]);
  a.T = static_cast<int>(c.rows(op.in[0]));
  a.pos0 = c.pos0;
  a.n_heads = op.iattr[1];
  a.n_kv = op.iattr[2];
  a.head_dim = static_cast<int>(c.tensor(op.in[0]).cols) / a.n_heads;
  EDGELM_CHECK(op.iattr[0] >= 0 && op.iattr[0] < static_cast<int>(c.kv.size()), "attention: bad layer");
  a.cache = c.kv[op.iattr[0]];
  a.rope = op.iattr[3] ? c.rope : nullptr;
  return a;
}

const float* f32_weight(const ExecContext& c, int i) { return static_cast<const float*>(c.tensor(i).data); }

// Shared by both host backends: the ops whose arithmetic does not depend on the backend.
bool run_common(const Op& op, ExecContext& c) {
  const int64_t n = c.rows(op.out[0]) * c.tensor(op.out[0]).cols;
  switch (op.type) {
    case OpType::ROPE:
      host::rope(c.f(op.in[0]), c.f(op.out[0]), static_cast<int>(c.rows(op.in[0])), op.iattr[0], op.iattr[1], c.pos0,
                 *c.rope);
      return true;
    case OpType::ADD: host::add(c.f(op.in[0]), c.f(op.in[1]), c.f(op.out[0]), n); return true;
    case OpType::SILU: host::silu(c.f(op.in[0]), c.f(op.out[0]), n); return true;
    case OpType::MUL: host::mul(c.f(op.in[0]), c.f(op.in[1]), c.f(op.out[0]), n); return true;
    default: return false;
  }
}

class ReferenceBackend : public Backend {
 public:
  const char* name() const override { return "reference"; }
  bool supports(const Graph&, const Op& op) const override { return !is_matmul_family(op.type); }
  void run(const Op& op, ExecContext& c) override {
    if (run_common(op, c)) return;
    switch (op.type) {
      case OpType::EMBED:
        host::embed(reinterpret_cast<const int32_t*>(c.f(op.in[0])), c.T, c.tensor(op.in[1]), c.f(op.out[0]));
        return;
      case OpType::RMSNORM:
        host::rmsnorm_ref(c.f(op.in[0]), f32_weight(c, op.in[1]), c.f(op.out[0]), static_cast<int>(c.rows(op.in[0])),
                          static_cast<int>(c.tensor(op.in[0]).cols), op.fattr[0]);
        return;
      case OpType::ATTENTION: host::attention_ref(attn_args(op, c)); return;
      case OpType::LAST_ROWS: {
        const int64_t cols = c.tensor(op.in[0]).cols, skip = c.rows(op.in[0]) - c.rows(op.out[0]);
        EDGELM_CHECK(skip >= 0, "LAST_ROWS: L > T");
        std::memmove(c.f(op.out[0]), c.f(op.in[0]) + skip * cols,
                     sizeof(float) * static_cast<size_t>(c.rows(op.out[0]) * cols));
        return;
      }
      default: EDGELM_CHECK(false, std::string("reference: unhandled op ") + op_name(op.type));
    }
  }
};

class CpuBackend : public Backend {
 public:
  const char* name() const override { return "cpu"; }
  bool supports(const Graph&, const Op& op) const override {
    return !is_matmul_family(op.type) && op.type != OpType::EMBED && op.type != OpType::LAST_ROWS;
  }
  void run(const Op& op, ExecContext& c) override {
    if (run_common(op, c)) return;
    switch (op.type) {
      case OpType::RMSNORM:
        host::rmsnorm(c.f(op.in[0]), f32_weight(c, op.in[1]), c.f(op.out[0]), static_cast<int>(c.rows(op.in[0])),
                      static_cast<int>(c.tensor(op.in[0]).cols), op.fattr[0], c.pool);
        return;
      case OpType::ATTENTION: host::attention(attn_args(op, c), c.pool); return;
      default: EDGELM_CHECK(false, std::string("cpu: unsupported op ") + op_name(op.type));
    }
  }
};

}  // namespace

std::unique_ptr<Backend> make_reference_backend() { return std::make_unique<ReferenceBackend>(); }
std::unique_ptr<Backend> make_cpu_backend() { return std::make_unique<CpuBackend>(); }

std::unique_ptr<Backend> make_backend(const std::string& name) {
  if (name == "reference" || name == "ref") return make_reference_backend();
  if (name == "cpu") return make_cpu_backend();
  if (name == "hip") return make_hip_backend(0);
  if (name == "hip-matmul") return make_hip_matmul_backend(0);
  throw std::runtime_error("edgelm: unknown backend " + name);
}

std::vector<Partition> partition_graph(const Graph& g, const std::vector<Backend*>& preference) {
  std::vector<Partition> parts;
  for (size_t i = 0; i < g.ops.size(); ++i) {
    Backend* owner = nullptr;
    for (Backend* b : preference)
      if (b->supports(g, g.ops[i])) {
        owner = b;
        break;
      }
    EDGELM_CHECK(owner, std::string("no backend supports ") + op_name(g.ops[i].type));
    if (!parts.empty() && parts.back().backend == owner) parts.back().end = static_cast<int>(i) + 1;
    else parts.push_back({owner, static_cast<int>(i), static_cast<int>(i) + 1});
  }
  return parts;
}

std::string describe_partitions(const Graph& g, const std::vector<Partition>& parts) {
  std::map<std::string, std::pair<int, int>> per;  // backend -> (partitions, ops)
  for (const Partition& p : parts) {
    auto& e = per[p.backend->name()];
    ++e.first;
    e.second += p.end - p.begin;
  }
  std::ostringstream os;
  os << parts.size() << " partitions:";
  for (const auto& kv : per) os << " " << kv.first << " " << kv.second.second << " ops in " << kv.second.first << ";";
  if (parts.size() <= 8)
    for (const Partition& p : parts) {
      os << "\n  [" << p.begin << ", " << p.end << ") " << p.backend->name() << ": " << op_name(g.ops[p.begin].type);
      if (p.end - p.begin > 1) os << " .. " << op_name(g.ops[p.end - 1].type);
    }
  return os.str();
}

}  // namespace edgelm

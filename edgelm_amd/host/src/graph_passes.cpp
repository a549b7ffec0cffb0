// Graph helpers, the four fusion passes and the activation memory planner. The fusion rules are
// edgelm's (passes.cpp:30-153): the fused graph has the same ops in the same order, so a session of
// this build computes the same thing as edgelm's on the same .elm file.
#include <algorithm>
#include <climits>
#include <map>
#include <sstream>

#include "edgelm/runtime.hpp"

namespace edgelm {

const char* op_name(OpType t) {
  switch (t) {
    case OpType::EMBED: return "EMBED";
    case OpType::RMSNORM: return "RMSNORM";
    case OpType::MATMUL: return "MATMUL";
    case OpType::ROPE: return "ROPE";
    case OpType::ATTENTION: return "ATTENTION";
    case OpType::ADD: return "ADD";
    case OpType::SILU: return "SILU";
    case OpType::MUL: return "MUL";
    case OpType::LAST_ROWS: return "LAST_ROWS";
    case OpType::MATMUL_N: return "MATMUL_N";
    case OpType::FFN_SWIGLU: return "FFN_SWIGLU";
    case OpType::MATMUL_ADD: return "MATMUL_ADD";
    default: return "?";
  }
}

const char* dtype_name(DType d) {
  switch (d) {
    case DType::F32: return "f32";
    case DType::Q8: return "q8";
    case DType::Q4: return "q4";
    case DType::I32: return "i32";
  }
  return "?";
}

void Graph::index_io() {
  input = output = -1;
  for (size_t i = 0; i < tensors.size(); ++i) {
    if (tensors[i].kind == TensorKind::Input) input = static_cast<int>(i);
    if (tensors[i].kind == TensorKind::Output) output = static_cast<int>(i);
  }
  EDGELM_CHECK(input >= 0 && output >= 0, "graph needs one input and one output tensor");
}

std::vector<std::vector<int>> Graph::consumers() const {
  std::vector<std::vector<int>> c(tensors.size());
  for (size_t i = 0; i < ops.size(); ++i)
    for (int t : ops[i].in) c[t].push_back(static_cast<int>(i));
  return c;
}

std::string Graph::summary() const {
  std::map<std::string, int> count;
  for (const Op& op : ops) ++count[op_name(op.type)];
  std::ostringstream os;
  os << ops.size() << " ops (";
  const char* sep = "";
  for (const auto& kv : count) {
    os << sep << kv.first << " " << kv.second;
    sep = ", ";
  }
  os << ")";
  return os.str();
}

namespace {

struct Maps {
  std::vector<int> producer;
  std::vector<std::vector<int>> consumers;
  explicit Maps(const Graph& g) : producer(g.tensors.size(), -1), consumers(g.consumers()) {
    for (size_t i = 0; i < g.ops.size(); ++i)
      for (int t : g.ops[i].out) producer[t] = static_cast<int>(i);
  }
  bool only(int tensor, int op) const { return consumers[tensor].size() == 1 && consumers[tensor][0] == op; }
};

void drop(Graph& g, const std::vector<char>& dead) {
  std::vector<Op> keep;
  keep.reserve(g.ops.size());
  for (size_t i = 0; i < g.ops.size(); ++i)
    if (!dead[i]) keep.push_back(std::move(g.ops[i]));
  g.ops.swap(keep);
}

}  // namespace

// MATMUL(gate), MATMUL(up), SILU(gate), MUL(silu, up) -> FFN_SWIGLU at the MUL's position.
int fuse_swiglu(Graph& g) {
  const Maps m(g);
  std::vector<char> dead(g.ops.size(), 0);
  int fused = 0;
  for (size_t i = 0; i < g.ops.size(); ++i) {
    if (g.ops[i].type != OpType::MUL) continue;
    for (int side = 0; side < 2; ++side) {
      const int act = g.ops[i].in[side], lin = g.ops[i].in[1 - side];
      const int si = m.producer[act], ui = m.producer[lin];
      if (si < 0 || ui < 0 || g.ops[si].type != OpType::SILU || g.ops[ui].type != OpType::MATMUL) continue;
      const int gi = m.producer[g.ops[si].in[0]];
      if (gi < 0 || g.ops[gi].type != OpType::MATMUL || g.ops[gi].in[0] != g.ops[ui].in[0]) continue;
      if (!m.only(act, static_cast<int>(i)) || !m.only(lin, static_cast<int>(i)) || !m.only(g.ops[si].in[0], si) ||
          dead[si] || dead[ui] || dead[gi])
        continue;
      Op f;
      f.type = OpType::FFN_SWIGLU;
      f.name = g.ops[i].name + "+swiglu";
      f.in = {g.ops[gi].in[0], g.ops[gi].in[1], g.ops[ui].in[1]};
      f.out = g.ops[i].out;
      dead[si] = dead[ui] = dead[gi] = 1;
      g.ops[i] = f;
      ++fused;
      break;
    }
  }
  drop(g, dead);
  return fused;
}

// MATMULs reading the same tensor -> one MATMUL_N at the earliest one's position.
int fuse_shared_input(Graph& g) {
  std::vector<char> dead(g.ops.size(), 0);
  int fused = 0;
  for (size_t i = 0; i < g.ops.size(); ++i) {
    if (dead[i] || g.ops[i].type != OpType::MATMUL) continue;
    const int x = g.ops[i].in[0];
    std::vector<size_t> group{i};
    for (size_t j = i + 1; j < g.ops.size(); ++j)
      if (!dead[j] && g.ops[j].type == OpType::MATMUL && g.ops[j].in[0] == x) group.push_back(j);
    if (group.size() < 2) continue;
    Op f;
    f.type = OpType::MATMUL_N;
    f.in = {x};
    for (size_t j : group) {
      f.in.push_back(g.ops[j].in[1]);
      f.out.push_back(g.ops[j].out[0]);
      if (!f.name.empty()) f.name += "+";
      f.name += g.ops[j].name;
      if (j != i) dead[j] = 1;
    }
    g.ops[i] = f;
    ++fused;
  }
  drop(g, dead);
  return fused;
}

// MATMUL then ADD(r, that) -> MATMUL_ADD at the ADD's position.
int fuse_residual(Graph& g) {
  const Maps m(g);
  std::vector<char> dead(g.ops.size(), 0);
  int fused = 0;
  for (size_t i = 0; i < g.ops.size(); ++i) {
    if (g.ops[i].type != OpType::ADD) continue;
    for (int side = 0; side < 2; ++side) {
      const int y = g.ops[i].in[side], r = g.ops[i].in[1 - side];
      const int mi = m.producer[y];
      if (mi < 0 || dead[mi] || g.ops[mi].type != OpType::MATMUL || !m.only(y, static_cast<int>(i))) continue;
      Op f;
      f.type = OpType::MATMUL_ADD;
      f.name = g.ops[mi].name + "+residual";
      f.in = {g.ops[mi].in[0], g.ops[mi].in[1], r};
      f.out = g.ops[i].out;
      dead[mi] = 1;
      g.ops[i] = f;
      ++fused;
      break;
    }
  }
  drop(g, dead);
  return fused;
}

// ROPE(q), ROPE(k) feeding only an ATTENTION -> ATTENTION with fused rope.
int fuse_rope_attention(Graph& g) {
  const Maps m(g);
  std::vector<char> dead(g.ops.size(), 0);
  int fused = 0;
  for (size_t i = 0; i < g.ops.size(); ++i) {
    Op& at = g.ops[i];
    if (at.type != OpType::ATTENTION || at.iattr[3]) continue;
    const int qi = m.producer[at.in[0]], ki = m.producer[at.in[1]];
    if (qi < 0 || ki < 0 || g.ops[qi].type != OpType::ROPE || g.ops[ki].type != OpType::ROPE) continue;
    if (!m.only(at.in[0], static_cast<int>(i)) || !m.only(at.in[1], static_cast<int>(i))) continue;
    at.in[0] = g.ops[qi].in[0];
    at.in[1] = g.ops[ki].in[0];
    at.iattr[3] = 1;
    at.name += "+rope";
    dead[qi] = dead[ki] = 1;
    ++fused;
  }
  drop(g, dead);
  return fused;
}

FusionStats optimize(Graph& g) {
  FusionStats s;
  s.ops_before = g.ops.size();
  s.swiglu = fuse_swiglu(g);  // first, so gate/up become one SwiGLU rather than a MATMUL_N
  s.shared_input = fuse_shared_input(g);
  s.residual = fuse_residual(g);
  s.rope = fuse_rope_attention(g);
  s.ops_after = g.ops.size();
  return s;
}

// Live range = [producing op, last consumer]; tensors placed largest first into the tightest gap
// among already-placed tensors whose ranges overlap (greedy by size), 64-byte aligned.
MemoryPlan plan_memory(const Graph& g, int T, int L) {
  constexpr int64_t kAlign = 64;
  const size_t nt = g.tensors.size();
  const int nops = static_cast<int>(g.ops.size());
  MemoryPlan p;
  p.offset.assign(nt, -1);
  p.bytes.assign(nt, 0);
  p.first.assign(nt, -1);
  p.last.assign(nt, -1);
  for (int i = 0; i < nops; ++i) {
    for (int t : g.ops[i].out)
      if (p.first[t] < 0) p.first[t] = i;
    for (int t : g.ops[i].in) p.last[t] = std::max(p.last[t], i);
  }
  std::vector<int> order;
  for (size_t t = 0; t < nt; ++t) {
    const Tensor& ts = g.tensors[t];
    if (ts.is_weight()) continue;
    if (ts.kind == TensorKind::Input) p.first[t] = 0;
    if (ts.kind == TensorKind::Output) p.last[t] = nops;
    if (p.first[t] < 0 || p.last[t] < 0) continue;
    const int64_t rows = ts.rows_sym == RowSym::T ? T : ts.rows_sym == RowSym::L ? L : ts.rows;
    p.bytes[t] = (rows * ts.cols * 4 + kAlign - 1) / kAlign * kAlign;
    p.naive_bytes += static_cast<size_t>(p.bytes[t]);
    order.push_back(static_cast<int>(t));
  }
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return p.bytes[a] > p.bytes[b]; });
  std::vector<int> placed;
  for (int t : order) {
    std::vector<std::pair<int64_t, int64_t>> busy;
    for (int o : placed)
      if (p.first[o] <= p.last[t] && p.first[t] <= p.last[o]) busy.emplace_back(p.offset[o], p.offset[o] + p.bytes[o]);
    std::sort(busy.begin(), busy.end());
    int64_t best = -1, best_gap = INT64_MAX, cur = 0;
    for (const auto& iv : busy) {
      const int64_t gap = iv.first - cur;
      if (gap >= p.bytes[t] && gap < best_gap) {
        best = cur;
        best_gap = gap;
      }
      cur = std::max(cur, iv.second);
    }
    p.offset[t] = best >= 0 ? best : cur;
    p.arena_bytes = std::max<size_t>(p.arena_bytes, static_cast<size_t>(p.offset[t] + p.bytes[t]));
    placed.push_back(t);
    ++p.n_planned;
  }
  return p;
}

bool plan_is_valid(const MemoryPlan& p) {
  const size_t n = p.offset.size();
  for (size_t a = 0; a < n; ++a) {
    if (p.offset[a] < 0) continue;
    if (p.offset[a] % 64 || p.offset[a] + p.bytes[a] > static_cast<int64_t>(p.arena_bytes)) return false;
    for (size_t b = a + 1; b < n; ++b) {
      if (p.offset[b] < 0) continue;
      const bool live = p.first[a] <= p.last[b] && p.first[b] <= p.last[a];
      const bool mem = p.offset[a] < p.offset[b] + p.bytes[b] && p.offset[b] < p.offset[a] + p.bytes[a];
      if (live && mem) return false;
    }
  }
  return true;
}

}  // namespace edgelm

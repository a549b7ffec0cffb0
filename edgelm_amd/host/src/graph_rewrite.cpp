// Graph IR helpers and the fusion rewrites that turn edgelm's exported Llama graph into the op types
// the hot path serves. The rewrites must produce what edgelm's passes produce (passes.cpp:30-153) —
// the same fused ops, each at a position that keeps the list a valid order — because a session of this
// runtime is compared with edgelm's own on the same file. Here every rewrite is a rule applied through
// a use-def view (Rewriter): a rule matches a pattern around one anchor op, replaces the anchor with
// the fused op and removes the ops it absorbed; the view compacts the list when the rule is done.
#include <map>
#include <sstream>
#include <stdexcept>

#include "edgelm/runtime.hpp"

namespace edgelm {

const char* op_name(OpType t) {
  constexpr const char* kNames[] = {"EMBED",     "RMSNORM",  "MATMUL",     "ROPE",      "ATTENTION", "ADD",
                                    "SILU",      "MUL",      "LAST_ROWS",  "MATMUL_N",  "FFN_SWIGLU", "MATMUL_ADD"};
  static_assert(sizeof(kNames) / sizeof(kNames[0]) == static_cast<size_t>(OpType::COUNT), "one name per op type");
  const auto i = static_cast<size_t>(t);
  return i < static_cast<size_t>(OpType::COUNT) ? kNames[i] : "?";
}

const char* dtype_name(DType d) {
  constexpr const char* kNames[] = {"f32", "q8", "q4", "i32"};
  const auto i = static_cast<size_t>(d);
  return i < 4 ? kNames[i] : "?";
}

void Graph::index_io() {
  input = output = -1;
  for (int i = 0; i < static_cast<int>(tensors.size()); ++i) {
    if (tensors[i].kind == TensorKind::Input) input = i;
    if (tensors[i].kind == TensorKind::Output) output = i;
  }
  if (input < 0 || output < 0) throw std::runtime_error("edgelm: a graph needs an input and an output tensor");
}

std::vector<std::vector<int>> Graph::consumers() const {
  std::vector<std::vector<int>> readers(tensors.size());
  for (int i = 0; i < static_cast<int>(ops.size()); ++i)
    for (int t : ops[i].in) readers[t].push_back(i);
  return readers;
}

std::string Graph::summary() const {
  std::map<std::string, int> hist;
  for (const Op& op : ops) ++hist[op_name(op.type)];
  std::ostringstream os;
  os << ops.size() << " ops (";
  for (auto it = hist.begin(); it != hist.end(); ++it) os << (it == hist.begin() ? "" : ", ") << it->first << " " << it->second;
  os << ")";
  return os.str();
}

namespace {

// Use-def view of g.ops for one rewrite rule: which op defines each tensor and how many operand slots
// read it (counted when the view is built). Ops are replaced in place or removed; finish() drops the
// removed ones, keeping the order of the rest.
class Rewriter {
 public:
  explicit Rewriter(Graph& g) : g_(g), def_(g.tensors.size(), -1), reads_(g.tensors.size(), 0), gone_(g.ops.size(), 0) {
    for (int i = 0; i < static_cast<int>(g.ops.size()); ++i) {
      for (int t : g.ops[i].out) def_[t] = i;
      for (int t : g.ops[i].in) ++reads_[t];
    }
  }
  int size() const { return static_cast<int>(g_.ops.size()); }
  const Op& op(int i) const { return g_.ops[i]; }
  Op& mutable_op(int i) { return g_.ops[i]; }
  bool alive(int i) const { return !gone_[i]; }
  // the live op of `type` that defines t, or -1
  int defined_by(int t, OpType type) const {
    const int i = def_[t];
    return i >= 0 && !gone_[i] && g_.ops[i].type == type ? i : -1;
  }
  // t is read by exactly one operand slot of the graph
  bool read_once(int t) const { return reads_[t] == 1; }
  void remove(int i) { gone_[i] = 1; }
  void replace(int i, Op fused) {
    g_.ops[i] = std::move(fused);
    ++rewrites_;
  }
  int finish() {
    size_t keep = 0;
    for (size_t i = 0; i < g_.ops.size(); ++i) {
      if (gone_[i]) continue;
      if (keep != i) g_.ops[keep] = std::move(g_.ops[i]);  // (a self-move would empty the op's vectors)
      ++keep;
    }
    g_.ops.resize(keep);
    return rewrites_;
  }

 private:
  Graph& g_;
  std::vector<int> def_, reads_;
  std::vector<char> gone_;
  int rewrites_ = 0;
};

Op make_op(OpType type, std::string name, std::vector<int> in, std::vector<int> out) {
  Op op;
  op.type = type;
  op.name = std::move(name);
  op.in = std::move(in);
  op.out = std::move(out);
  return op;
}

}  // namespace

// MUL(SILU(MATMUL(x, Wg)), MATMUL(x, Wu)), every intermediate read once -> FFN_SWIGLU(x, Wg, Wu) in the
// MUL's place.
int fuse_swiglu(Graph& g) {
  Rewriter rw(g);
  for (int i = 0; i < rw.size(); ++i) {
    if (rw.op(i).type != OpType::MUL) continue;
    for (int side : {0, 1}) {
      const int act = rw.op(i).in[side], lin = rw.op(i).in[1 - side];
      const int s = rw.defined_by(act, OpType::SILU), u = rw.defined_by(lin, OpType::MATMUL);
      if (s < 0 || u < 0) continue;
      const int gate = rw.op(s).in[0], gm = rw.defined_by(gate, OpType::MATMUL);
      if (gm < 0 || rw.op(gm).in[0] != rw.op(u).in[0]) continue;
      if (!rw.read_once(act) || !rw.read_once(lin) || !rw.read_once(gate)) continue;
      const Op& mul = rw.op(i);
      Op f = make_op(OpType::FFN_SWIGLU, mul.name + "+swiglu", {rw.op(gm).in[0], rw.op(gm).in[1], rw.op(u).in[1]}, mul.out);
      rw.remove(s);
      rw.remove(u);
      rw.remove(gm);
      rw.replace(i, std::move(f));
      break;
    }
  }
  return rw.finish();
}

// MATMULs reading the same input -> one MATMUL_N (targets in op order) in the first one's place.
int fuse_shared_input(Graph& g) {
  Rewriter rw(g);
  std::map<int, std::vector<int>> by_input;  // input tensor -> its MATMULs in order
  std::vector<int> first_seen;
  for (int i = 0; i < rw.size(); ++i) {
    if (rw.op(i).type != OpType::MATMUL) continue;
    auto& v = by_input[rw.op(i).in[0]];
    if (v.empty()) first_seen.push_back(rw.op(i).in[0]);
    v.push_back(i);
  }
  for (int x : first_seen) {
    const std::vector<int>& group = by_input[x];
    if (group.size() < 2) continue;
    Op f = make_op(OpType::MATMUL_N, "", {x}, {});
    for (int j : group) {
      f.in.push_back(rw.op(j).in[1]);
      f.out.push_back(rw.op(j).out[0]);
      f.name += (f.name.empty() ? "" : "+") + rw.op(j).name;
      if (j != group.front()) rw.remove(j);
    }
    rw.replace(group.front(), std::move(f));
  }
  return rw.finish();
}

// ADD(r, MATMUL(x, W)) (either operand order, the MATMUL's output read once) -> MATMUL_ADD(x, W, r) in the
// ADD's place.
int fuse_residual(Graph& g) {
  Rewriter rw(g);
  for (int i = 0; i < rw.size(); ++i) {
    if (rw.op(i).type != OpType::ADD) continue;
    for (int side : {0, 1}) {
      const int y = rw.op(i).in[side], r = rw.op(i).in[1 - side];
      const int m = rw.defined_by(y, OpType::MATMUL);
      if (m < 0 || !rw.read_once(y)) continue;
      Op f = make_op(OpType::MATMUL_ADD, rw.op(m).name + "+residual", {rw.op(m).in[0], rw.op(m).in[1], r}, rw.op(i).out);
      rw.remove(m);
      rw.replace(i, std::move(f));
      break;
    }
  }
  return rw.finish();
}

// ATTENTION(ROPE(q), ROPE(k), v), both rotated tensors read once -> ATTENTION(q, k, v) rotating inside
// (iattr[3] = 1).
int fuse_rope_attention(Graph& g) {
  Rewriter rw(g);
  int fused = 0;
  for (int i = 0; i < rw.size(); ++i) {
    const Op& at = rw.op(i);
    if (at.type != OpType::ATTENTION || at.iattr[3]) continue;
    const int rq = rw.defined_by(at.in[0], OpType::ROPE), rk = rw.defined_by(at.in[1], OpType::ROPE);
    if (rq < 0 || rk < 0 || !rw.read_once(at.in[0]) || !rw.read_once(at.in[1])) continue;
    Op& a = rw.mutable_op(i);
    a.in[0] = rw.op(rq).in[0];
    a.in[1] = rw.op(rk).in[0];
    a.iattr[3] = 1;
    a.name += "+rope";
    rw.remove(rq);
    rw.remove(rk);
    ++fused;
  }
  rw.finish();
  return fused;
}

FusionStats optimize(Graph& g) {
  FusionStats s;
  s.ops_before = g.ops.size();
  // SwiGLU first: gate and up read the same input and would otherwise become a MATMUL_N
  s.swiglu = fuse_swiglu(g);
  s.shared_input = fuse_shared_input(g);
  s.residual = fuse_residual(g);
  s.rope = fuse_rope_attention(g);
  s.ops_after = g.ops.size();
  return s;
}

}  // namespace edgelm

// Activation arena planning: every non-weight tensor gets an offset in one host buffer, and two tensors
// share bytes only if their live ranges (producing op .. last reading op) do not overlap. The reference
// places tensors greedily by size (passes.cpp:160-204); this planner is a linear scan over the ops
// instead: walking the op list once, it returns a tensor's block to a free list after its last reader
// and gives each new output the smallest free block that holds it (best fit), growing the arena only
// when none does. Offsets and sizes are multiples of 64 bytes.
#include <algorithm>
#include <map>

#include "edgelm/runtime.hpp"

namespace edgelm {
namespace {

constexpr int64_t kArenaAlign = 64;

// Free blocks of the arena, by offset; neighbours merge when a block is returned.
class FreeBlocks {
 public:
  int64_t take(int64_t bytes) {
    auto best = blocks_.end();
    for (auto it = blocks_.begin(); it != blocks_.end(); ++it)
      if (it->second >= bytes && (best == blocks_.end() || it->second < best->second)) best = it;
    if (best == blocks_.end()) {
      // nothing fits: extend the arena, starting inside a free block that ends at its top
      int64_t at = top_;
      if (!blocks_.empty()) {
        auto last = std::prev(blocks_.end());
        if (last->first + last->second == top_) {
          at = last->first;
          blocks_.erase(last);
        }
      }
      top_ = at + bytes;
      return at;
    }
    const int64_t at = best->first, rest = best->second - bytes;
    blocks_.erase(best);
    if (rest > 0) blocks_[at + bytes] = rest;
    return at;
  }
  void give_back(int64_t at, int64_t bytes) {
    auto it = blocks_.emplace(at, bytes).first;
    auto next = std::next(it);
    if (next != blocks_.end() && it->first + it->second == next->first) {
      it->second += next->second;
      blocks_.erase(next);
    }
    if (it != blocks_.begin()) {
      auto prev = std::prev(it);
      if (prev->first + prev->second == it->first) {
        prev->second += it->second;
        blocks_.erase(it);
      }
    }
  }
  int64_t top() const { return top_; }

 private:
  std::map<int64_t, int64_t> blocks_;
  int64_t top_ = 0;
};

}  // namespace

MemoryPlan plan_memory(const Graph& g, int T, int L) {
  const int nt = static_cast<int>(g.tensors.size()), nops = static_cast<int>(g.ops.size());
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
  // births[i]: tensors first written by op i; deaths[i]: tensors last read by op i
  std::vector<std::vector<int>> births(nops + 1), deaths(nops + 1);
  for (int t = 0; t < nt; ++t) {
    const Tensor& ts = g.tensors[t];
    if (ts.is_weight()) continue;
    if (ts.kind == TensorKind::Input) p.first[t] = 0;     // written by the caller before op 0
    if (ts.kind == TensorKind::Output) p.last[t] = nops;  // read by the caller after the last op
    if (p.first[t] < 0 || p.last[t] < 0) continue;       // not used by the (fused) graph
    const int64_t rows = ts.rows_sym == RowSym::T ? T : ts.rows_sym == RowSym::L ? L : ts.rows;
    p.bytes[t] = (rows * ts.cols * 4 + kArenaAlign - 1) / kArenaAlign * kArenaAlign;
    p.naive_bytes += static_cast<size_t>(p.bytes[t]);
    births[p.first[t]].push_back(t);
    deaths[p.last[t]].push_back(t);
  }
  FreeBlocks arena;
  for (int i = 0; i <= nops; ++i) {
    // the outputs of op i may not reuse what op i still reads: place them first, free after
    std::vector<int>& born = births[i];
    std::stable_sort(born.begin(), born.end(), [&](int a, int b) { return p.bytes[a] > p.bytes[b]; });
    for (int t : born) {
      p.offset[t] = arena.take(p.bytes[t]);
      ++p.n_planned;
    }
    for (int t : deaths[i]) arena.give_back(p.offset[t], p.bytes[t]);
  }
  p.arena_bytes = static_cast<size_t>(arena.top());
  return p;
}

bool plan_is_valid(const MemoryPlan& p) {
  // sweep the planned tensors by offset: each must end inside the arena, sit on a 64-byte boundary, and
  // not share bytes with any tensor whose live range overlaps its own
  std::vector<int> order;
  for (int t = 0; t < static_cast<int>(p.offset.size()); ++t)
    if (p.offset[t] >= 0) order.push_back(t);
  std::sort(order.begin(), order.end(), [&](int a, int b) { return p.offset[a] < p.offset[b]; });
  for (size_t i = 0; i < order.size(); ++i) {
    const int a = order[i];
    if (p.offset[a] % kArenaAlign || p.offset[a] + p.bytes[a] > static_cast<int64_t>(p.arena_bytes)) return false;
    for (size_t j = i + 1; j < order.size() && p.offset[order[j]] < p.offset[a] + p.bytes[a]; ++j) {
      const int b = order[j];
      if (p.first[a] <= p.last[b] && p.first[b] <= p.last[a]) return false;
    }
  }
  return true;
}

}  // namespace edgelm

// The MI355X delegate as an edgelm Backend (reference interface backend.hpp:30-36; template
// MatmulOnlyBackend, backends.cpp:137-150), in two flavours:
//   "hip"         MATMUL, MATMUL_N, MATMUL_ADD, FFN_SWIGLU (q8 or q4 weights) and the rest of a
//                 layer: EMBED (q8/q4 table), RMSNORM, ATTENTION (RoPE and KV cache on the
//                 device) and LAST_ROWS;
//   "hip-matmul"  the matmul family only (the cpu backend runs the rest).
//
// With prepare() (an optional hook this build's Backend adds; edgelm's Backend lacks it, so there it
// is simply never called) activations stay in HBM between consecutive hip ops: prepare() marks which
// activation tensors hip ops produce and which another backend reads or the graph outputs, and
// run() uploads an input produced on the host once per forward, keeps every output on the device
// and copies an output into the host arena only when the host needs it. Without prepare(), as
// inside an unmodified edgelm Session, run() uploads every input and copies every output back.
// Either way the host has what it needs when run() returns (edgelm's contract: runtime.cpp:66-76).
// Weights are uploaded to HBM once, on first use (matmul weights repacked; RMSNORM weights f32).
//
// run_partition() (another optional hook) replays a decode step (T = 1) of a whole partition of
// at least kMinGraphOps ops as one HIP graph: the first such step runs op by op (allocating
// buffers and uploading weights), the second is captured, with attention reading the position
// from device memory; every later step uploads the host-side inputs (token ids) and the
// position, launches the graph, and copies back what the host reads (the logits). Prefill
// forwards (T > 1) replay graphs the same way, one per (partition, T, first position), since
// their kernels take the length and the position as arguments; at most kMaxPrefillGraphs are
// kept. A buffer that has to grow (a longer prefill) drops the graphs. EDGELM_HIP_GRAPHS=0 turns
// graphs off, EDGELM_HIP_PREFILL_GRAPHS=0 the prefill graphs only.
//
// keep_output() and argmax_output() (the greedy-sampling hooks) leave the logits in HBM and hand
// the host only the argmax of their last row.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <tuple>
#include <unordered_map>

#include "edgelm/backend.hpp"
#include "elmh.h"

namespace edgelm {
namespace {

bool matmul_family(OpType t) {
  return t == OpType::MATMUL || t == OpType::MATMUL_N || t == OpType::MATMUL_ADD || t == OpType::FFN_SWIGLU;
}

class HipBackend : public Backend {
 public:
  // device < 0: planning only (supports() answers, run() throws) — for partition inspection on a
  // host without a GPU.
  HipBackend(int device, bool layer_ops) : layer_ops_(layer_ops) {
    const char* g = std::getenv("EDGELM_HIP_GRAPHS");
    graphs_on_ = !(g && g[0] == '0');
    const char* pg = std::getenv("EDGELM_HIP_PREFILL_GRAPHS");
    prefill_graphs_on_ = !(pg && pg[0] == '0');
    if (device < 0) return;
    if (elmh_create(device, &ctx_) != ELMH_OK)
      throw std::runtime_error(std::string("edgelm: hip backend unavailable: ") + elmh_last_error(nullptr));
  }
  ~HipBackend() override {
    if (!ctx_) return;
    drop_graphs();
    elmh_free(ctx_, pos_dev_);
    for (auto& kv : weights_) elmh_free_weight(ctx_, kv.second);
    for (auto& kv : f32w_) elmh_free(ctx_, kv.second);
    for (Buf& b : act_) elmh_free(ctx_, b.p);
    for (Layer& l : kv_) {
      elmh_free(ctx_, l.k);
      elmh_free(ctx_, l.v);
    }
    elmh_free(ctx_, rope_cos_);
    elmh_free(ctx_, rope_sin_);
    elmh_free(ctx_, dev_tok_);
    elmh_free(ctx_, step_ring_);
    release_pins();
    elmh_destroy(ctx_);
  }

  const char* name() const override { return layer_ops_ ? "hip" : "hip-matmul"; }

  bool supports(const Graph& g, const Op& op) const override {
    if (matmul_family(op.type)) {
      const size_t count = op.type == OpType::MATMUL_N ? op.out.size() : op.type == OpType::FFN_SWIGLU ? 2 : 1;
      if (op.in.size() < 1 + count) return false;
      for (size_t i = 1; i <= count; ++i)
        if (!quantized(g.tensors[op.in[i]])) return false;
      return true;
    }
    if (!layer_ops_) return false;
    switch (op.type) {
      case OpType::EMBED: return op.in.size() == 2 && quantized(g.tensors[op.in[1]]);
      case OpType::RMSNORM: {
        const Tensor& w = g.tensors[op.in[1]];
        return w.is_weight() && w.dtype == DType::F32 && g.tensors[op.in[0]].cols <= 16384;
      }
      case OpType::ATTENTION: {
        const int nh = op.iattr[1], nkv = op.iattr[2];
        if (nh < 1 || nkv < 1 || nh % nkv) return false;
        const int64_t hd = g.tensors[op.in[0]].cols / nh;
        return hd >= 4 && hd % 4 == 0 && hd <= 256;
      }
      case OpType::LAST_ROWS: return true;
      default: return false;
    }
  }

  void prepare(const Graph& g, const std::vector<Partition>& parts) {  // overrides where Backend declares it
    const size_t nt = g.tensors.size();
    on_dev_.assign(nt, 0);
    host_needed_.assign(nt, 0);
    for (const Partition& p : parts)
      for (int i = p.begin; i < p.end; ++i) {
        const Op& op = g.ops[i];
        if (p.backend == this) {
          for (int t : op.out) on_dev_[t] = 1;
        } else {
          for (int t : op.in) host_needed_[t] = 1;
        }
      }
    if (g.output >= 0) host_needed_[g.output] = 1;
    output_ = g.output >= 0 && on_dev_[g.output] ? g.output : -1;
    // RMSNORM whose output only feeds the matmul right after it, both here: one fused call
    std::vector<int> readers(nt, 0);
    for (const Op& op : g.ops)
      for (int t : op.in) ++readers[t];
    fuse_norm_.assign(g.ops.size(), 0);
    fuse_attn_.assign(g.ops.size(), 0);
    fuse_ffn_.assign(g.ops.size(), 0);
    for (const Partition& p : parts) {
      if (p.backend != this) continue;
      for (int i = p.begin; i + 1 < p.end; ++i) {
        const Op &a = g.ops[i], &b = g.ops[i + 1];
        const int t = a.type == OpType::RMSNORM ? a.out[0] : -1;
        fuse_norm_[i] = t >= 0 && !host_needed_[t] && readers[t] == 1 && !b.in.empty() && b.in[0] == t &&
                        (b.type == OpType::MATMUL || b.type == OpType::MATMUL_N || b.type == OpType::MATMUL_ADD ||
                         b.type == OpType::FFN_SWIGLU);
        // ATTENTION whose output the next op (the o projection) multiplies: one call, which still
        // writes the attention output for later device readers (none on the host: its copy-back
        // would run before the deferred kernel)
        fuse_attn_[i] = a.type == OpType::ATTENTION && !host_needed_[a.out[0]] && !b.in.empty() &&
                        b.in[0] == a.out[0] && (b.type == OpType::MATMUL || b.type == OpType::MATMUL_ADD);
        // FFN_SWIGLU whose output h only the next op (the down projection) multiplies: one call, in
        // which the SwiGLU launch can hand h over quantized (it still writes h)
        fuse_ffn_[i] = a.type == OpType::FFN_SWIGLU && !host_needed_[a.out[0]] && readers[a.out[0]] == 1 &&
                       !b.in.empty() && b.in[0] == a.out[0] && (b.type == OpType::MATMUL || b.type == OpType::MATMUL_ADD);
      }
    }
    act_.assign(nt, Buf{});
    release_pins();
    pin_.assign(nt, Pin{});
    first_op_ = -1;
    for (const Partition& p : parts)
      if (p.backend == this && (first_op_ < 0 || p.begin < first_op_)) first_op_ = p.begin;
    prepared_ = true;
  }

  // overrides where Backend declares it; false: the Session runs the partition op by op
  bool run_partition(const Partition& p, ExecContext& c) {
    // a graph launch costs ~100 us of host time: only long partitions gain from replaying one
    if (!graphs_on_ || !ctx_ || !prepared_ || c.L != 1 || p.end - p.begin < kMinGraphOps) return false;
    const bool step = c.T == 1;
    if (!step && !prefill_graphs_on_) return false;
    const Graph& g = *c.graph;
    const auto pkey = std::make_tuple(p.begin, c.T, c.pos0);
    if (!step && prefill_.size() >= kMaxPrefillGraphs && !prefill_.count(pkey)) drop_prefill_graphs();
    StepGraph& sg = step ? graphs_[p.begin] : prefill_[pkey];
    if (step && sg.warm == 0) {
      // a captured step reads its position from device memory and sizes attention's score row for the
      // whole cache; past the kernel's limit the partition runs op by op, sized by the position in use
      for (int i = p.begin; i < p.end; ++i) {
        const Op& op = g.ops[i];
        if (op.type != OpType::ATTENTION || op.iattr[0] < 0 || op.iattr[0] >= static_cast<int>(c.kv.size())) continue;
        const int hd = static_cast<int>(c.tensor(op.in[0]).cols) / std::max(op.iattr[1], 1);
        if (!elmh_attention_step_supported(hd, c.kv[op.iattr[0]].max_ctx)) sg.eager = true;
      }
    }
    if (sg.eager) return false;
    if (!sg.exec && sg.warm == 0) {  // warm-up: allocations and uploads happen op by op
      for (int i = p.begin; i < p.end; ++i) run(g.ops[i], c);
      sg.warm = 1;
      return true;
    }
    step_checks(p, c);
    upload_step_inputs(p, c);
    if (sg.exec && sg.scratch_gen != elmh_scratch_generation(ctx_)) {
      // the library's scratch moved since the capture (a larger op ran in between): capture again
      elmh_graph_destroy(ctx_, sg.exec);
      sg.exec = nullptr;
    }
    if (!sg.exec) {
      capturing_ = true;
      const uint64_t gen = buffer_gen_;
      int rc = elmh_graph_begin(ctx_);
      if (rc == ELMH_OK) {
        try {
          for (int i = p.begin; i < p.end; ++i) run(g.ops[i], c);
        } catch (...) {
          void* dead = nullptr;
          elmh_graph_end(ctx_, &dead);
          if (dead) elmh_graph_destroy(ctx_, dead);
          capturing_ = false;
          throw;
        }
        rc = elmh_graph_end(ctx_, &sg.exec);
      }
      capturing_ = false;
      if (rc != ELMH_OK) throw std::runtime_error(std::string("edgelm: hip graph capture: ") + elmh_last_error(ctx_));
      if (gen != buffer_gen_) throw std::runtime_error("edgelm: hip graph capture: a buffer moved while capturing");
      sg.scratch_gen = elmh_scratch_generation(ctx_);
    }
    if (elmh_graph_launch(ctx_, sg.exec) != ELMH_OK)
      throw std::runtime_error(std::string("edgelm: hip graph launch: ") + elmh_last_error(ctx_));
    for (int i = p.begin; i < p.end; ++i)
      for (int t : g.ops[i].out)
        if (to_host(t)) download(t, c);
    flush();
    return true;
  }

  void run(const Op& op, ExecContext& c) override {
    if (!ctx_) throw std::runtime_error("edgelm: hip backend created for planning only");
    if (!prepared_) unprepared(*c.graph);
    const int idx = static_cast<int>(&op - c.graph->ops.data());
    // a new upload epoch before any input is read (a fresh buffer has epoch 0, so it is uploaded): once per
    // forward with prepare(), and for every op without it (no residency: every op uploads its inputs)
    if (idx == first_op_ || !prepared_) ++epoch_;
    // a deferred RMSNORM (fuse_norm_) applies to this op's input inside the matmul call
    const bool normed = norm_.op == idx - 1 && norm_.op >= 0;
    if (!normed) norm_.op = -1;
    // a deferred ATTENTION (fuse_attn_) runs inside this matmul's call
    const bool attended = attn_.op == idx - 1 && attn_.op >= 0;
    if (!attended) attn_.op = -1;
    // a deferred FFN_SWIGLU (fuse_ffn_) runs inside this matmul's call
    const bool ffned = ffn_.op == idx - 1 && ffn_.op >= 0;
    if (!ffned) ffn_.op = -1;
    switch (op.type) {
      case OpType::FFN_SWIGLU: {
        const int T = static_cast<int>(c.rows(op.in[0]));
        const int64_t K = c.tensor(op.in[1]).cols;
        if (prepared_ && fuse_ffn_[idx]) {
          ffn_ = {idx, normed ? norm_.x : in(op.in[0], c), normed ? norm_.w : nullptr, normed ? norm_.eps : 0.f, T, K,
                  c.tensor(op.in[1]).rows, weight(c.tensor(op.in[1])), weight(c.tensor(op.in[2])), out(op.out[0], c)};
          return;  // the next op (the down projection) runs it
        }
        if (normed)
          check(elmh_rmsnorm_swiglu_dev(ctx_, norm_.x, norm_.w, norm_.eps, T, K, weight(c.tensor(op.in[1])),
                                        weight(c.tensor(op.in[2])), out(op.out[0], c), act(c), ELMH_EXACT),
                op);
        else
          check(elmh_swiglu_dev(ctx_, in(op.in[0], c), T, K, weight(c.tensor(op.in[1])), weight(c.tensor(op.in[2])),
                                out(op.out[0], c), act(c), ELMH_EXACT),
                op);
        break;
      }
      case OpType::MATMUL:
      case OpType::MATMUL_N:
      case OpType::MATMUL_ADD: {
        const int T = static_cast<int>(c.rows(op.in[0]));
        const int64_t K = c.tensor(op.in[1]).cols;
        const size_t n = op.type == OpType::MATMUL_N ? op.out.size() : 1;
        w_.resize(n);
        y_.resize(n);
        r_.assign(n, nullptr);
        const float* x = normed ? nullptr : in(op.in[0], c);
        for (size_t i = 0; i < n; ++i) {
          w_[i] = weight(c.tensor(op.in[1 + i]));
          y_[i] = out(op.out[i], c);
        }
        if (op.type == OpType::MATMUL_ADD) r_[0] = in(op.in[2], c);
        const float* const* res = op.type == OpType::MATMUL_ADD ? r_.data() : nullptr;
        if (normed)
          check(elmh_rmsnorm_matmul_dev(ctx_, norm_.x, norm_.w, norm_.eps, T, K, static_cast<int>(n), w_.data(),
                                        y_.data(), res, act(c), ELMH_EXACT),
                op);
        else if (ffned) {
          const PendingFfn& f = ffn_;
          EDGELM_CHECK(n == 1 && f.h == x && f.T == T && f.N == K, "ffn + matmul: operands do not match");
          check(elmh_ffn_dev(ctx_, f.x, f.nw, f.eps, f.T, f.K, f.wg, f.wu, f.h, w_[0], y_[0], r_[0], act(c), ELMH_EXACT),
                op);
          ffn_.op = -1;
        } else if (attended) {
          const PendingAttention& a = attn_;
          EDGELM_CHECK(n == 1 && a.out == x && a.T == T && static_cast<int64_t>(a.nh) * a.hd == K,
                       "attention + matmul: operands do not match");
          check(elmh_attention_matmul_dev(ctx_, a.q, a.k, a.v, a.out, T, a.pos0, a.nh, a.nkv, a.hd, a.kc, a.vc, a.mc,
                                          a.rc, a.rs, w_[0], y_[0], r_[0], act(c), ELMH_EXACT),
                op);
          attn_.op = -1;
        } else
          check(elmh_matmul_dev(ctx_, x, T, K, static_cast<int>(n), w_.data(), y_.data(), res, act(c), ELMH_EXACT),
                op);
        break;
      }
      case OpType::EMBED: {
        const Tensor& table = c.tensor(op.in[1]);
        const int32_t* tok = reinterpret_cast<const int32_t*>(c.f(op.in[0]));
        for (int t = 0; t < c.T; ++t)
          EDGELM_CHECK(tok[t] >= 0 && tok[t] < table.rows, "token id out of range");
        check(elmh_embed_dev(ctx_, reinterpret_cast<const int32_t*>(in(op.in[0], c)), c.T, weight(table),
                             out(op.out[0], c)),
              op);
        break;
      }
      case OpType::RMSNORM: {
        const int rows = static_cast<int>(c.rows(op.in[0])), dim = static_cast<int>(c.tensor(op.in[0]).cols);
        if (prepared_ && fuse_norm_[idx] && dim <= kMaxFusedNormDim) {
          norm_ = {idx, in(op.in[0], c), f32_weight(c.tensor(op.in[1])), op.fattr[0]};
          return;  // the next op runs it; its output is read by nothing else
        }
        check(elmh_rmsnorm_dev(ctx_, in(op.in[0], c), f32_weight(c.tensor(op.in[1])), out(op.out[0], c), rows, dim,
                               op.fattr[0]),
              op);
        break;
      }
      case OpType::ATTENTION: attention(op, c); break;
      case OpType::LAST_ROWS: {
        const int64_t cols = c.tensor(op.in[0]).cols, skip = c.rows(op.in[0]) - c.rows(op.out[0]);
        EDGELM_CHECK(skip >= 0, "LAST_ROWS: L > T");
        const float* src = in(op.in[0], c) + skip * cols;
        check(elmh_memcpy_d2d(ctx_, out(op.out[0], c), src, bytes(op.out[0], c)), op);
        break;
      }
      default: throw std::runtime_error(std::string("edgelm: hip: unsupported op ") + op_name(op.type));
    }
    if (capturing_) return;  // the replay copies host-needed outputs after the launch
    for (int t : op.out)
      if (to_host(t)) download(t, c);
    flush();
  }

  // greedy sampling: the logits stay in HBM and only the token id crosses to the host
  bool keep_output(bool on) {  // overrides where Backend declares it
    keep_out_ = on && ctx_ && prepared_ && output_ >= 0;
    return keep_out_;
  }
  bool argmax_output(const ExecContext& c, int32_t* tok) {  // overrides where Backend declares it
    if (!keep_out_ || !act_[output_].p) return false;
    if (!dev_tok_ && elmh_malloc(ctx_, sizeof(int32_t), reinterpret_cast<void**>(&dev_tok_)) != ELMH_OK)
      throw std::runtime_error(std::string("edgelm: hip argmax: ") + elmh_last_error(ctx_));
    const int64_t V = c.tensor(output_).cols, rows = c.rows(output_);
    const float* last = static_cast<const float*>(act_[output_].p) + (rows - 1) * V;
    if (elmh_argmax_dev(ctx_, last, 1, V, dev_tok_) != ELMH_OK || elmh_memcpy_d2h(ctx_, tok, dev_tok_, sizeof(int32_t)) != ELMH_OK)
      throw std::runtime_error(std::string("edgelm: hip argmax: ") + elmh_last_error(ctx_));
    synced();  // a synchronous copy: every earlier transfer has completed
    return true;
  }

  // Greedy decode steps queued back to back: once the step graph is captured, each step is the
  // graph's launch and one argmax launch, which writes the token id straight into the buffer the
  // next step's EMBED reads, bumps the device position the next step's attention reads and keeps
  // the id in a device ring; the host copies the ring back and waits once per kStepRing steps and
  // at the end. Until the graph exists, steps run one by one with their token on the host.
  bool greedy_steps(const Partition& p, ExecContext& c, int32_t first, int n, int32_t* out) {  // overrides where Backend declares it
    const Graph& g = *c.graph;
    if (!graphs_on_ || !ctx_ || !prepared_ || !keep_out_ || output_ < 0 || g.input < 0 || c.L != 1 || n < 1 ||
        p.begin != 0 || p.end != static_cast<int>(g.ops.size()))
      return false;
    for (size_t t = 0; t < host_needed_.size(); ++t)
      if (host_needed_[t] && static_cast<int>(t) != output_) return false;  // another reader of an activation
    const int pos0 = c.pos0;
    int32_t tok = first;
    int i = 0;
    auto ready = [&]() {
      auto it = graphs_.find(p.begin);
      return it != graphs_.end() && it->second.exec && !it->second.eager &&
             it->second.scratch_gen == elmh_scratch_generation(ctx_);
    };
    for (; i < n && !ready(); ++i) {  // one by one: warm-up, capture
      std::memcpy(c.f(g.input), &tok, sizeof tok);
      c.T = 1;
      c.pos0 = pos0 + i;
      if (!run_partition(p, c))
        for (int k = p.begin; k < p.end; ++k) run(g.ops[k], c);
      if (!argmax_output(c, &tok)) throw std::runtime_error("edgelm: hip greedy: the logits are not on the device");
      out[i] = tok;
    }
    if (i == n) return true;
    // the replayed steps' token ids come from the device argmax (in range by construction); the first
    // one may still be the caller's, so it gets run()'s check here
    for (int k = p.begin; k < p.end; ++k)
      if (g.ops[k].type == OpType::EMBED)
        EDGELM_CHECK(tok >= 0 && tok < c.tensor(g.ops[k].in[1]).rows, "token id out of range");
    StepGraph& sg = graphs_[p.begin];
    // pinned staging: the ring's copy [kStepRing], then the first replayed step's token and position
    const size_t need = kStepRing + 2;
    if (step_pin_cap_ < need) {
      wait_all();
      elmh_host_free(ctx_, step_pin_);
      step_pin_ = nullptr;
      step_pin_cap_ = 0;
      if (elmh_host_alloc(ctx_, need * sizeof(int32_t), reinterpret_cast<void**>(&step_pin_)) != ELMH_OK)
        throw std::runtime_error(std::string("edgelm: hip pinned staging: ") + elmh_last_error(ctx_));
      step_pin_cap_ = need;
    }
    if (!step_ring_ && elmh_malloc(ctx_, kStepRing * sizeof(int32_t), reinterpret_cast<void**>(&step_ring_)) != ELMH_OK)
      throw std::runtime_error(std::string("edgelm: hip: ") + elmh_last_error(ctx_));
    int32_t* const d_tok = static_cast<int32_t*>(act_[g.input].p);  // the EMBED's token ids
    const int64_t V = c.tensor(output_).cols;
    const float* const logits = static_cast<const float*>(act_[output_].p);
    auto ok = [&](int rc) {
      if (rc != ELMH_OK) throw std::runtime_error(std::string("edgelm: hip greedy steps: ") + elmh_last_error(ctx_));
    };
    wait_all();  // earlier copies out of the staging buffer are done
    // the device carries the steps from here: each step's argmax writes the next step's token id
    // where its EMBED reads it, bumps the position its attention reads, and leaves the id in a ring
    // slot (position mod kStepRing) that the host collects every kStepRing steps
    step_pin_[kStepRing] = tok;
    step_pin_[kStepRing + 1] = pos0 + i;
    ok(elmh_memcpy_h2d_async(ctx_, d_tok, step_pin_ + kStepRing, sizeof(int32_t)));
    ok(elmh_memcpy_h2d_async(ctx_, pos_dev_, step_pin_ + kStepRing + 1, sizeof(int32_t)));
    for (int done = i; i < n; ++i) {
      c.pos0 = pos0 + i;
      for (int k = p.begin; k < p.end; ++k) {  // run()'s position checks for a replayed step
        const Op& op = g.ops[k];
        if (op.type == OpType::ATTENTION) {
          EDGELM_CHECK(c.pos0 + 1 <= c.kv[op.iattr[0]].max_ctx, "context overflow");
          EDGELM_CHECK(!op.iattr[3] || c.pos0 + 1 <= rope_pos_, "position beyond rope table");
        }
      }
      ok(elmh_graph_launch(ctx_, sg.exec));
      ok(elmh_argmax_step_dev(ctx_, logits, V, d_tok, pos_dev_, step_ring_, kStepRing));
      if (i + 1 - done == kStepRing || i + 1 == n) {  // the ring holds every step since `done`
        ok(elmh_memcpy_d2h_async(ctx_, step_pin_, step_ring_, kStepRing * sizeof(int32_t)));
        ok(elmh_synchronize(ctx_));
        for (int k = done; k <= i; ++k) out[k] = step_pin_[(pos0 + k) & (kStepRing - 1)];
        done = i + 1;
      }
    }
    return true;
  }

 private:
  static constexpr int kStepRing = 64;  // a power of two
  int32_t* step_pin_ = nullptr;  // pinned: the ring's copy, the first replayed step's token and position
  size_t step_pin_cap_ = 0;
  int32_t* step_ring_ = nullptr;  // device: greedy steps' token ids by position mod kStepRing

  bool to_host(int t) const { return host_needed_[t] && !(keep_out_ && t == output_); }

  // Host <-> device transfers of activations go through pinned staging buffers, one per tensor, as
  // stream-ordered copies: an op's uploads, kernels and downloads are enqueued together and waited
  // for once (flush). A staging buffer still used by a copy in flight is reused only after a wait.
  struct Pin {
    void* p = nullptr;
    size_t cap = 0;
    bool busy = false;  // an async copy may still read or write it
  };
  struct Download {
    Pin* pin;
    void* host;
    size_t n;
  };
  void synced() {
    for (Pin* b : busy_) b->busy = false;
    busy_.clear();
  }
  void wait_all() {
    if (busy_.empty()) return;
    if (elmh_synchronize(ctx_) != ELMH_OK) throw std::runtime_error(std::string("edgelm: hip sync: ") + elmh_last_error(ctx_));
    synced();
  }
  void* staging(Pin& b, size_t n) {
    if (b.busy) wait_all();
    if (n > b.cap) {
      elmh_host_free(ctx_, b.p);
      b.p = nullptr;
      b.cap = 0;
      if (elmh_host_alloc(ctx_, n, &b.p) != ELMH_OK)
        throw std::runtime_error(std::string("edgelm: hip pinned staging: ") + elmh_last_error(ctx_));
      b.cap = n;
    }
    return b.p;
  }
  void upload(Pin& b, void* dev, const void* host, size_t n) {
    void* h = staging(b, n);
    std::memcpy(h, host, n);
    if (elmh_memcpy_h2d_async(ctx_, dev, h, n) != ELMH_OK)
      throw std::runtime_error(std::string("edgelm: hip upload: ") + elmh_last_error(ctx_));
    b.busy = true;
    busy_.push_back(&b);
  }
  void download(int t, const ExecContext& c) {
    const size_t n = bytes(t, c);
    void* h = staging(pin_[t], n);
    if (elmh_memcpy_d2h_async(ctx_, h, act_[t].p, n) != ELMH_OK)
      throw std::runtime_error(std::string("edgelm: hip download: ") + elmh_last_error(ctx_));
    pin_[t].busy = true;
    busy_.push_back(&pin_[t]);
    downs_.push_back({&pin_[t], c.f(t), n});
  }
  void flush() {  // wait for the enqueued downloads and move them into the host arena
    if (downs_.empty()) return;
    wait_all();
    for (const Download& d : downs_) std::memcpy(d.host, d.pin->p, d.n);
    downs_.clear();
  }
  void release_pins() {
    if (!ctx_) return;
    if (!busy_.empty()) elmh_synchronize(ctx_);
    synced();
    downs_.clear();
    for (Pin& b : pin_) elmh_host_free(ctx_, b.p);
    pin_.clear();
    elmh_host_free(ctx_, pin_pos_.p);
    pin_pos_ = Pin{};
    elmh_host_free(ctx_, step_pin_);
    step_pin_ = nullptr;
    step_pin_cap_ = 0;
  }
  struct Buf {
    void* p = nullptr;
    size_t cap = 0;
    uint64_t epoch = 0;  // forward in which a host-produced tensor was last uploaded
  };
  struct Layer {
    float* k = nullptr;
    float* v = nullptr;
  };
  // Partitions of a few ops (the hip-matmul flavour's, between host-run ops) gain less from one
  // graph launch than the launch itself costs: they run op by op.
  static constexpr int kMinGraphOps = 16;
  struct StepGraph {
    int warm = 0;
    void* exec = nullptr;
    uint64_t scratch_gen = 0;  // elmh_scratch_generation at capture
    bool eager = false;        // never captured: an attention op's cache is past the step kernel's limit
  };

  void drop_graphs() {
    for (auto& kv : graphs_)
      if (kv.second.exec) elmh_graph_destroy(ctx_, kv.second.exec);
    graphs_.clear();
    drop_prefill_graphs();
  }
  void drop_prefill_graphs() {
    for (auto& kv : prefill_)
      if (kv.second.exec) elmh_graph_destroy(ctx_, kv.second.exec);
    prefill_.clear();
  }
  // what run() checks on the host each time, for a replayed step: token ids and positions in range
  void step_checks(const Partition& p, const ExecContext& c) const {
    const Graph& g = *c.graph;
    for (int i = p.begin; i < p.end; ++i) {
      const Op& op = g.ops[i];
      if (op.type == OpType::EMBED) {
        const int32_t* tok = reinterpret_cast<const int32_t*>(c.f(op.in[0]));
        for (int t = 0; t < c.T; ++t)
          EDGELM_CHECK(tok[t] >= 0 && tok[t] < c.tensor(op.in[1]).rows, "token id out of range");
      } else if (op.type == OpType::ATTENTION) {
        EDGELM_CHECK(c.pos0 + c.T <= c.kv[op.iattr[0]].max_ctx, "context overflow");
        EDGELM_CHECK(!op.iattr[3] || c.pos0 + c.T <= rope_pos_, "position beyond rope table");
      }
    }
  }
  // a replayed step's inputs that come from the host (token ids; anything another backend made)
  // and the position the graph's attention reads
  void upload_step_inputs(const Partition& p, const ExecContext& c) {
    const Graph& g = *c.graph;
    for (int i = p.begin; i < p.end; ++i)
      for (int t : g.ops[i].in)
        if (!c.tensor(t).is_weight() && !on_dev_[t]) upload(pin_[t], act_[t].p, c.f(t), bytes(t, c));
    bool attn = false;
    for (int i = p.begin; i < p.end; ++i) attn = attn || g.ops[i].type == OpType::ATTENTION;
    if (!attn) return;
    if (!pos_dev_) pos_dev_ = static_cast<int32_t*>(alloc(sizeof(int32_t)));
    const int32_t pos = c.pos0;
    upload(pin_pos_, pos_dev_, &pos, sizeof pos);
  }

  // no prepare() call (an edgelm Session without the hook): nothing is known to be on the device
  // and the host may read every output
  void unprepared(const Graph& g) {
    if (act_.size() == g.tensors.size()) return;
    on_dev_.assign(g.tensors.size(), 0);
    host_needed_.assign(g.tensors.size(), 1);
    act_.assign(g.tensors.size(), Buf{});
    release_pins();
    pin_.assign(g.tensors.size(), Pin{});
    first_op_ = -1;
  }

  static bool quantized(const Tensor& w) {
    return w.is_weight() && (w.dtype == DType::Q8 || (w.dtype == DType::Q4 && w.cols % 32 == 0));
  }
  int act(const ExecContext& c) const { return c.act_quant ? ELMH_ACT_INT8 : ELMH_ACT_F32; }
  void check(int rc, const Op& op) const {
    if (rc != ELMH_OK) throw std::runtime_error(std::string("edgelm: hip ") + op_name(op.type) + ": " + elmh_last_error(ctx_));
  }
  size_t bytes(int t, const ExecContext& c) const {
    return static_cast<size_t>(c.rows(t) * c.tensor(t).cols) * sizeof(float);
  }
  void* alloc(size_t n) {
    void* p = nullptr;
    if (elmh_malloc(ctx_, n, &p) != ELMH_OK) throw std::runtime_error(std::string("edgelm: hip: ") + elmh_last_error(ctx_));
    return p;
  }
  // device buffer of activation t, large enough for this forward's rows
  float* buffer(int t, const ExecContext& c) {
    Buf& b = act_[t];
    const size_t n = bytes(t, c);
    if (b.cap < n) {
      if (capturing_) throw std::runtime_error("edgelm: hip: buffer growth during graph capture");
      if (b.p) {
        elmh_free(ctx_, b.p);
        drop_graphs();  // captured graphs hold the old address
        ++buffer_gen_;
      }
      b.p = alloc(n);
      b.cap = n;
      b.epoch = 0;
    }
    return static_cast<float*>(b.p);
  }
  float* out(int t, const ExecContext& c) { return buffer(t, c); }
  // an input on the device: produced there by an earlier hip op, or uploaded from the host arena
  // (once per forward)
  const float* in(int t, const ExecContext& c) {
    float* p = buffer(t, c);
    if (!on_dev_[t] && !capturing_ && act_[t].epoch != epoch_) {
      upload(pin_[t], p, c.f(t), bytes(t, c));
      act_[t].epoch = epoch_;
    }
    return p;
  }

  elmh_weight* weight(const Tensor& t) {
    auto it = weights_.find(&t);
    if (it != weights_.end()) return it->second;
    elmh_weight* w = nullptr;
    const int dt = static_cast<int>(t.dtype);
#ifdef EDGELM_TENSOR_DEVICE_IMAGE
    // the weight already in the device layout (a device image attached to the model)
    const int rc = t.image ? elmh_upload_weight_image(ctx_, dt, t.rows, t.cols, t.image, t.image_scales, &w)
                           : elmh_upload_weight(ctx_, dt, t.rows, t.cols, t.data, t.scales, &w);
#else
    const int rc = elmh_upload_weight(ctx_, dt, t.rows, t.cols, t.data, t.scales, &w);
#endif
    if (rc != ELMH_OK)
      throw std::runtime_error(std::string("edgelm: hip upload of ") + t.name + ": " + elmh_last_error(ctx_));
    weights_.emplace(&t, w);
    return w;
  }
  const float* f32_weight(const Tensor& t) {
    auto it = f32w_.find(&t);
    if (it != f32w_.end()) return static_cast<const float*>(it->second);
    const size_t n = static_cast<size_t>(t.rows * t.cols) * sizeof(float);
    void* p = alloc(n);
    if (elmh_memcpy_h2d(ctx_, p, t.data, n) != ELMH_OK)
      throw std::runtime_error(std::string("edgelm: hip upload of ") + t.name + ": " + elmh_last_error(ctx_));
    f32w_.emplace(&t, p);
    return static_cast<const float*>(p);
  }

  // cpu::attention's arguments (backends.cpp attn_args) with the cache and the rope table in HBM
  void attention(const Op& op, ExecContext& c) {
    const int layer = op.iattr[0], nh = op.iattr[1], nkv = op.iattr[2];
    EDGELM_CHECK(layer >= 0 && layer < static_cast<int>(c.kv.size()), "attention: bad layer");
    const int T = static_cast<int>(c.rows(op.in[0]));
    const int hd = static_cast<int>(c.tensor(op.in[0]).cols) / nh;
    const int mc = c.kv[layer].max_ctx;
    if (kv_.size() < c.kv.size()) kv_.resize(c.kv.size());
    Layer& l = kv_[layer];
    if (!l.k) {
      const size_t n = static_cast<size_t>(nkv) * mc * hd * sizeof(float);
      l.k = static_cast<float*>(alloc(n));
      l.v = static_cast<float*>(alloc(n));
      check(elmh_memset_dev(ctx_, l.k, 0, n), op);
      check(elmh_memset_dev(ctx_, l.v, 0, n), op);
    }
    const float *rc = nullptr, *rs = nullptr;
    if (op.iattr[3]) {
      EDGELM_CHECK(c.rope && c.rope->half * 2 == hd, "attention: rope table does not match head_dim");
      if (!rope_cos_) {
        const size_t n = c.rope->cos.size() * sizeof(float);
        rope_cos_ = static_cast<float*>(alloc(n));
        rope_sin_ = static_cast<float*>(alloc(n));
        check(elmh_memcpy_h2d(ctx_, rope_cos_, c.rope->cos.data(), n), op);
        check(elmh_memcpy_h2d(ctx_, rope_sin_, c.rope->sin.data(), n), op);
        rope_pos_ = c.rope->max_pos;
      }
      EDGELM_CHECK(c.pos0 + T <= rope_pos_, "position beyond rope table");
      rc = rope_cos_;
      rs = rope_sin_;
    }
    const float* q = in(op.in[0], c);
    const float* k = in(op.in[1], c);
    const float* v = in(op.in[2], c);
    const int idx = static_cast<int>(&op - c.graph->ops.data());
    if (prepared_ && fuse_attn_[idx] && !capturing_ && T > 1) {
      attn_ = {idx, q, k, v, out(op.out[0], c), T, c.pos0, nh, nkv, hd, l.k, l.v, mc, rc, rs};
      return;  // the next op (the o projection) runs it
    }
    if (capturing_)  // the replayed step reads its position from device memory
      check(elmh_attention_step_dev(ctx_, q, k, v, out(op.out[0], c), pos_dev_, nh, nkv, hd, l.k, l.v, mc, rc, rs), op);
    else
      check(elmh_attention_dev(ctx_, q, k, v, out(op.out[0], c), T, c.pos0, nh, nkv, hd, l.k, l.v, mc, rc, rs), op);
  }

  bool layer_ops_;
  bool graphs_on_ = true;
  bool capturing_ = false;
  uint64_t buffer_gen_ = 0;
  std::map<int, StepGraph> graphs_;  // by the partition's first op
  // prefill forwards (T > 1) replayed as graphs, by (the partition's first op, T, first position):
  // their kernels take the length and the position as arguments
  bool prefill_graphs_on_ = true;
  static constexpr size_t kMaxPrefillGraphs = 8;
  std::map<std::tuple<int, int, int>, StepGraph> prefill_;
  int32_t* pos_dev_ = nullptr;
  elmh_ctx* ctx_ = nullptr;
  bool prepared_ = false;
  int first_op_ = -1;
  uint64_t epoch_ = 0;
  std::vector<char> on_dev_, host_needed_;
  std::vector<char> fuse_norm_;  // op index: an RMSNORM that the next op (a matmul) applies
  struct PendingNorm {
    int op = -1;
    const float* x = nullptr;
    const float* w = nullptr;
    float eps = 0.f;
  } norm_;
  static constexpr int kMaxFusedNormDim = 8192;  // elmh_rmsnorm_matmul_dev's limit
  std::vector<char> fuse_attn_;  // op index: an ATTENTION that the next op (a matmul) runs
  struct PendingAttention {
    int op = -1;
    const float *q = nullptr, *k = nullptr, *v = nullptr;
    float* out = nullptr;
    int T = 0, pos0 = 0, nh = 0, nkv = 0, hd = 0;
    float *kc = nullptr, *vc = nullptr;
    int mc = 0;
    const float *rc = nullptr, *rs = nullptr;
  } attn_;
  std::vector<char> fuse_ffn_;  // op index: an FFN_SWIGLU that the next op (a matmul) runs
  struct PendingFfn {
    int op = -1;
    const float* x = nullptr;   // the FFN's input, or RMSNORM's when nw is set
    const float* nw = nullptr;  // a deferred RMSNORM's weight
    float eps = 0.f;
    int T = 0;
    int64_t K = 0, N = 0;  // FFN_SWIGLU's input width and output width (the rows of gate and up)
    const elmh_weight *wg = nullptr, *wu = nullptr;
    float* h = nullptr;
  } ffn_;
  int output_ = -1;          // graph output when this backend writes it (prepare), else -1
  bool keep_out_ = false;    // keep_output(true): the output is not copied to the host arena
  int32_t* dev_tok_ = nullptr;  // argmax result
  std::vector<Pin> pin_;           // staging per activation tensor
  Pin pin_pos_;                    // staging of the decode position
  std::vector<Pin*> busy_;         // staging buffers of copies in flight
  std::vector<Download> downs_;    // downloads awaiting flush()
  std::vector<Buf> act_;
  std::vector<Layer> kv_;
  float* rope_cos_ = nullptr;
  float* rope_sin_ = nullptr;
  int rope_pos_ = 0;
  std::unordered_map<const Tensor*, elmh_weight*> weights_;
  std::unordered_map<const Tensor*, void*> f32w_;
  std::vector<elmh_weight*> w_;
  std::vector<float*> y_;
  std::vector<const float*> r_;
};

}  // namespace

std::unique_ptr<Backend> make_hip_backend(int device) { return std::make_unique<HipBackend>(device, true); }
std::unique_ptr<Backend> make_hip_matmul_backend(int device) { return std::make_unique<HipBackend>(device, false); }
std::unique_ptr<Backend> make_hip_planning_backend(bool layer_ops) { return std::make_unique<HipBackend>(-1, layer_ops); }

}  // namespace edgelm

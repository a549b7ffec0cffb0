// The MI355X delegate as an edgelm Backend (reference interface backend.hpp:30-36; template
// MatmulOnlyBackend, backends.cpp:137-150). It claims MATMUL, MATMUL_N, MATMUL_ADD and FFN_SWIGLU
// when every weight of the op is q8 or q4, uploads each weight tensor to HBM once (repacked) on
// first use, and runs the op through the C ABI of include/elmh.h. run() is synchronous: outputs
// are in the host arena when it returns, as edgelm's Session requires (runtime.cpp:66-76).
#include <unordered_map>

#include "edgelm/backend.hpp"
#include "elmh.h"

namespace edgelm {
namespace {

class HipBackend : public Backend {
 public:
  // device < 0: planning only (supports() answers, run() throws) — for partition inspection on a
  // host without a GPU.
  explicit HipBackend(int device) {
    if (device < 0) return;
    if (elmh_create(device, &ctx_) != ELMH_OK)
      throw std::runtime_error(std::string("edgelm: hip backend unavailable: ") + elmh_last_error(nullptr));
  }
  ~HipBackend() override {
    for (auto& kv : weights_) elmh_free_weight(ctx_, kv.second);
    if (ctx_) elmh_destroy(ctx_);
  }

  const char* name() const override { return "hip"; }

  bool supports(const Graph& g, const Op& op) const override {
    size_t first = 1, count = 0;
    switch (op.type) {
      case OpType::MATMUL:
      case OpType::MATMUL_ADD: count = 1; break;
      case OpType::MATMUL_N: count = op.out.size(); break;
      case OpType::FFN_SWIGLU: count = 2; break;
      default: return false;
    }
    if (op.in.size() < first + count) return false;
    for (size_t i = first; i < first + count; ++i) {
      const Tensor& w = g.tensors[op.in[i]];
      if (!w.is_weight() || (w.dtype != DType::Q8 && w.dtype != DType::Q4)) return false;
      if (w.dtype == DType::Q4 && w.cols % 32) return false;
    }
    return true;
  }

  void run(const Op& op, ExecContext& c) override {
    if (!ctx_) throw std::runtime_error("edgelm: hip backend created for planning only");
    const int T = static_cast<int>(c.rows(op.in[0]));
    const int64_t K = c.tensor(op.in[1]).cols;
    const int act = c.act_quant ? ELMH_ACT_INT8 : ELMH_ACT_F32;
    int rc = ELMH_OK;
    if (op.type == OpType::FFN_SWIGLU) {
      rc = elmh_swiglu(ctx_, c.f(op.in[0]), T, K, weight(c.tensor(op.in[1])), weight(c.tensor(op.in[2])),
                       c.f(op.out[0]), act, ELMH_EXACT);
    } else {
      const size_t n = op.type == OpType::MATMUL_N ? op.out.size() : 1;
      w_.resize(n);
      y_.resize(n);
      r_.assign(n, nullptr);
      for (size_t i = 0; i < n; ++i) {
        w_[i] = weight(c.tensor(op.in[1 + i]));
        y_[i] = c.f(op.out[i]);
      }
      if (op.type == OpType::MATMUL_ADD) r_[0] = c.f(op.in[2]);
      rc = elmh_matmul(ctx_, c.f(op.in[0]), T, K, static_cast<int>(n), w_.data(), y_.data(),
                       op.type == OpType::MATMUL_ADD ? r_.data() : nullptr, act, ELMH_EXACT);
    }
    if (rc != ELMH_OK) throw std::runtime_error(std::string("edgelm: hip ") + op_name(op.type) + ": " + elmh_last_error(ctx_));
  }

 private:
  elmh_weight* weight(const Tensor& t) {
    auto it = weights_.find(&t);
    if (it != weights_.end()) return it->second;
    elmh_weight* w = nullptr;
    if (elmh_upload_weight(ctx_, static_cast<int>(t.dtype), t.rows, t.cols, t.data, t.scales, &w) != ELMH_OK)
      throw std::runtime_error(std::string("edgelm: hip upload of ") + t.name + ": " + elmh_last_error(ctx_));
    weights_.emplace(&t, w);
    return w;
  }

  elmh_ctx* ctx_ = nullptr;
  std::unordered_map<const Tensor*, elmh_weight*> weights_;
  std::vector<elmh_weight*> w_;
  std::vector<float*> y_;
  std::vector<const float*> r_;
};

}  // namespace

std::unique_ptr<Backend> make_hip_backend(int device) { return std::make_unique<HipBackend>(device); }
std::unique_ptr<Backend> make_hip_planning_backend() { return std::make_unique<HipBackend>(-1); }

}  // namespace edgelm

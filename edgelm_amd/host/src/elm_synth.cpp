// Seeded random-init models in the .elm container, for the tests and the benchmark (no checkpoints
// are available offline). The graph is the unfused Llama decoder edgelm's exporter emits
// (tools/elm.py:105-161: EMBED, per layer RMSNORM / MATMUL q,k,v / ROPE q,k / ATTENTION / MATMUL o /
// ADD / RMSNORM / MATMUL gate,up / SILU / MUL / MATMUL down / ADD, then LAST_ROWS, RMSNORM and the LM
// head), built here from a table of one layer's steps; edgelm's own loader and fusion passes read
// the files (tests/test_host_runtime.py). Weight matrices are quantized with this library's q8 / q4
// quantizers, byte-identical to edgelm's.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "edgelm/elm_container.hpp"
#include "edgelm/graph.hpp"
#include "edgelm_host.h"

namespace edgelm {
namespace {

// ---- random numbers: splitmix64 streams, one per (seed, tensor, row), and the Box-Muller transform
// (computed in double, rounded to float), so every row is generated independently of thread count

uint64_t splitmix(uint64_t& s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

void normal_row(uint64_t seed, uint64_t tensor, uint64_t row, float mean, float sd, float* out, int64_t n) {
  uint64_t s = seed ^ (tensor * 0xD1B54A32D192ED03ull) ^ (row * 0xABC98388FB8FAC03ull);
  splitmix(s);
  constexpr double kTwoPi = 6.283185307179586;
  for (int64_t i = 0; i < n; i += 2) {
    const double u1 = (static_cast<double>(splitmix(s) >> 11) + 1.0) * 0x1p-53;  // (0, 1]
    const double u2 = static_cast<double>(splitmix(s) >> 11) * 0x1p-53;
    const double r = std::sqrt(-2.0 * std::log(u1));
    out[i] = static_cast<float>(mean + sd * r * std::cos(kTwoPi * u2));
    if (i + 1 < n) out[i + 1] = static_cast<float>(mean + sd * r * std::sin(kTwoPi * u2));
  }
}

template <class F>
void over_rows(int64_t rows, int threads, F&& body) {
  threads = std::max(1, std::min<int>(threads, static_cast<int>(std::min<int64_t>(rows, 64))));
  std::vector<std::thread> pool;
  for (int t = 0; t < threads; ++t)
    pool.emplace_back([&, t] {
      for (int64_t r = t; r < rows; r += threads) body(r);
    });
  for (auto& th : pool) th.join();
}

// ---- the container being assembled

struct PendingTensor {
  std::string name;
  TensorRecord rec{};
};
struct PendingOp {
  OpType type;
  std::string name;
  std::vector<int> in, out;
  OpAttrs attrs{};
};

class ContainerBuilder {
 public:
  int activation(const std::string& name, int64_t cols, RowSym rows = RowSym::T, TensorKind kind = TensorKind::Activation,
                 DType dt = DType::F32) {
    PendingTensor t;
    t.name = name;
    t.rec.kind = static_cast<uint8_t>(kind);
    t.rec.dtype = static_cast<uint8_t>(dt);
    t.rec.rows_sym = static_cast<uint8_t>(rows);
    t.rec.cols = cols;
    tensors_.push_back(t);
    return static_cast<int>(tensors_.size()) - 1;
  }
  // a weight array and, for q8 / q4, its scales, appended to the blob at 64-byte boundaries
  int weight(const std::string& name, DType dt, int64_t rows, int64_t cols, std::vector<uint8_t> data,
             std::vector<uint8_t> scales) {
    PendingTensor t;
    t.name = name;
    t.rec.kind = static_cast<uint8_t>(TensorKind::Weight);
    t.rec.dtype = static_cast<uint8_t>(dt);
    t.rec.rows_sym = static_cast<uint8_t>(RowSym::Const);
    t.rec.rows = rows;
    t.rec.cols = cols;
    t.rec.group = dt == DType::Q8 ? static_cast<uint32_t>(cols) : dt == DType::Q4 ? 32u : 0u;
    t.rec.data_off = append(data);
    t.rec.data_len = data.size();
    if (!scales.empty()) {
      t.rec.scale_off = append(scales);
      t.rec.scale_len = scales.size();
    }
    tensors_.push_back(t);
    return static_cast<int>(tensors_.size()) - 1;
  }
  void op(OpType type, const std::string& name, std::vector<int> in, std::vector<int> out, std::vector<int32_t> iattr = {},
          std::vector<float> fattr = {}) {
    PendingOp o{type, name, std::move(in), std::move(out), {}};
    std::copy(iattr.begin(), iattr.end(), o.attrs.iattr);
    std::copy(fattr.begin(), fattr.end(), o.attrs.fattr);
    ops_.push_back(std::move(o));
  }

  void write(const std::string& path, ContainerHeader h) const {
    std::vector<uint8_t> graph, tok;
    auto put = [](std::vector<uint8_t>& b, const void* p, size_t n) {
      const auto* c = static_cast<const uint8_t*>(p);
      b.insert(b.end(), c, c + n);
    };
    auto put_name = [&](std::vector<uint8_t>& b, const std::string& s) {
      const uint16_t n = static_cast<uint16_t>(s.size());
      put(b, &n, 2);
      put(b, s.data(), n);
    };
    for (const PendingTensor& t : tensors_) {
      put_name(graph, t.name);
      put(graph, &t.rec, sizeof t.rec);
    }
    for (const PendingOp& o : ops_) {
      const OpRecord r{static_cast<uint8_t>(o.type), static_cast<uint8_t>(o.in.size()), static_cast<uint8_t>(o.out.size()), 0};
      put(graph, &r, sizeof r);
      for (int id : o.in) put(graph, &id, 4);
      for (int id : o.out) put(graph, &id, 4);
      put(graph, &o.attrs, sizeof o.attrs);
      put_name(graph, o.name);
    }
    // tokenizer section: one single-byte token per id and no merges (the runs feed token ids)
    const uint32_t vocab = h.vocab, pretok = 1, merges = 0;
    put(tok, &vocab, 4);
    put(tok, &pretok, 4);
    for (uint32_t i = 0; i < vocab; ++i) {
      const uint8_t entry[4] = {1, 0, static_cast<uint8_t>(i & 0xFF), 0};  // u16 length 1, the byte, not special
      put(tok, entry, 4);
    }
    put(tok, &merges, 4);

    std::memcpy(h.magic, kElmMagic, 4);
    h.version = kElmVersion;
    h.n_tensors = static_cast<uint32_t>(tensors_.size());
    h.n_ops = static_cast<uint32_t>(ops_.size());
    h.graph = {sizeof(ContainerHeader), graph.size()};
    h.tok = {h.graph.off + h.graph.len, tok.size()};
    const uint64_t blob_off = (h.tok.off + h.tok.len + kElmAlign - 1) / kElmAlign * kElmAlign;
    h.blob = {blob_off, blob_.size()};
    std::unique_ptr<FILE, int (*)(FILE*)> f(std::fopen(path.c_str(), "wb"), &std::fclose);
    if (!f) throw std::runtime_error("edgelm: cannot create " + path);
    const std::vector<uint8_t> gap(blob_off - (h.tok.off + h.tok.len), 0);
    bool ok = std::fwrite(&h, sizeof h, 1, f.get()) == 1;
    const std::vector<uint8_t>* parts[] = {&graph, &tok, &gap, &blob_};
    for (const std::vector<uint8_t>* part : parts)
      ok = ok && (part->empty() || std::fwrite(part->data(), part->size(), 1, f.get()) == 1);
    if (!ok || std::fflush(f.get()) != 0) throw std::runtime_error("edgelm: writing " + path + " failed");
  }

 private:
  uint64_t append(const std::vector<uint8_t>& bytes) {
    blob_.resize((blob_.size() + kElmAlign - 1) / kElmAlign * kElmAlign, 0);
    const uint64_t at = blob_.size();
    blob_.insert(blob_.end(), bytes.begin(), bytes.end());
    return at;
  }
  std::vector<PendingTensor> tensors_;
  std::vector<PendingOp> ops_;
  std::vector<uint8_t> blob_;
};

// ---- one decoder layer as a table of steps. Operands name the layer input "x", activations made
// by earlier steps, or a weight by its Hugging Face suffix (a leading '#'). Widths: D = dim,
// H = hidden, Q = n_heads * head_dim, KV = n_kv_heads * head_dim.

enum Width { W_D, W_H, W_Q, W_KV };
enum Attr { A_NONE, A_NORM, A_ROPE_Q, A_ROPE_K, A_ATTN };
struct Step {
  OpType type;
  const char* op;
  const char* in[3];
  const char* out;
  Width width;
  Attr attr;
};

const Step kLayerSteps[] = {
    {OpType::RMSNORM, "attn_norm", {"x", "#input_layernorm.weight"}, "attn_in", W_D, A_NORM},
    {OpType::MATMUL, "wq", {"attn_in", "#self_attn.q_proj.weight"}, "q", W_Q, A_NONE},
    {OpType::MATMUL, "wk", {"attn_in", "#self_attn.k_proj.weight"}, "k", W_KV, A_NONE},
    {OpType::MATMUL, "wv", {"attn_in", "#self_attn.v_proj.weight"}, "v", W_KV, A_NONE},
    {OpType::ROPE, "rope_q", {"q"}, "q_rope", W_Q, A_ROPE_Q},
    {OpType::ROPE, "rope_k", {"k"}, "k_rope", W_KV, A_ROPE_K},
    {OpType::ATTENTION, "attention", {"q_rope", "k_rope", "v"}, "attn", W_Q, A_ATTN},
    {OpType::MATMUL, "wo", {"attn", "#self_attn.o_proj.weight"}, "attn_out", W_D, A_NONE},
    {OpType::ADD, "residual_attn", {"x", "attn_out"}, "x_attn", W_D, A_NONE},
    {OpType::RMSNORM, "ffn_norm", {"x_attn", "#post_attention_layernorm.weight"}, "ffn_in", W_D, A_NORM},
    {OpType::MATMUL, "w_gate", {"ffn_in", "#mlp.gate_proj.weight"}, "gate", W_H, A_NONE},
    {OpType::MATMUL, "w_up", {"ffn_in", "#mlp.up_proj.weight"}, "up", W_H, A_NONE},
    {OpType::SILU, "silu", {"gate"}, "gate_silu", W_H, A_NONE},
    {OpType::MUL, "gate_mul", {"gate_silu", "up"}, "ffn_mid", W_H, A_NONE},
    {OpType::MATMUL, "w_down", {"ffn_mid", "#mlp.down_proj.weight"}, "ffn_out", W_D, A_NONE},
    {OpType::ADD, "residual_ffn", {"x_attn", "ffn_out"}, "x_out", W_D, A_NONE},
};
constexpr const char* kLayerOutput = "x_out";

class Synth {
 public:
  explicit Synth(const elm_model_spec& s) : s_(s) {
    wdt_ = static_cast<DType>(s.weight_dtype);
    edt_ = s.embed_dtype < 0 ? wdt_ : static_cast<DType>(s.embed_dtype);
    for (DType d : {wdt_, edt_})
      if (d != DType::F32 && d != DType::Q8 && d != DType::Q4) throw std::runtime_error("edgelm: weight dtype must be f32, q8 or q4");
  }

  void build(const std::string& path) {
    const int64_t D = s_.dim, V = s_.vocab;
    const int tokens = b_.activation("tokens", 1, RowSym::T, TensorKind::Input, DType::I32);
    const int emb = matrix("model.embed_tokens.weight", V, D, edt_, s_.embed_sd);
    int x = b_.activation("x.embed", D);
    b_.op(OpType::EMBED, "embed", {tokens, emb}, {x});
    for (int l = 0; l < s_.n_layers; ++l) x = layer(l, x);
    const int last = b_.activation("x.last", D, RowSym::L);
    b_.op(OpType::LAST_ROWS, "last_rows", {x}, {last});
    const int fin = b_.activation("x.final_norm", D, RowSym::L);
    b_.op(OpType::RMSNORM, "final_norm", {last, norm("model.norm.weight")}, {fin}, {}, {s_.norm_eps});
    const int head = s_.tied ? emb : matrix("lm_head.weight", V, D, wdt_, s_.sd);
    const int logits = b_.activation("logits", V, RowSym::L, TensorKind::Output);
    b_.op(OpType::MATMUL, "lm_head", {fin, head}, {logits});

    ContainerHeader h{};
    h.vocab = static_cast<uint32_t>(s_.vocab);
    h.dim = static_cast<uint32_t>(s_.dim);
    h.hidden = static_cast<uint32_t>(s_.hidden);
    h.n_layers = static_cast<uint32_t>(s_.n_layers);
    h.n_heads = static_cast<uint32_t>(s_.n_heads);
    h.n_kv_heads = static_cast<uint32_t>(s_.n_kv_heads);
    h.head_dim = static_cast<uint32_t>(s_.head_dim);
    h.max_seq = static_cast<uint32_t>(s_.max_seq);
    h.rope_theta = s_.rope_theta;
    h.norm_eps = s_.norm_eps;
    h.bos = static_cast<uint32_t>(s_.bos);
    h.eos = static_cast<uint32_t>(s_.eos);
    h.weight_dtype = static_cast<uint32_t>(wdt_);
    h.group = wdt_ == DType::Q4 ? 32u : 0u;
    h.flags = s_.tied ? kElmFlagTied : 0u;
    b_.write(path, h);
  }

 private:
  int64_t width(Width w) const {
    switch (w) {
      case W_D: return s_.dim;
      case W_H: return s_.hidden;
      case W_Q: return static_cast<int64_t>(s_.n_heads) * s_.head_dim;
      default: return static_cast<int64_t>(s_.n_kv_heads) * s_.head_dim;
    }
  }
  // shape of a layer weight from the activations it connects: [out width, in width]
  int layer_weight(const std::string& name, int in_tensor, Width out) {
    return matrix(name, width(out), in_cols_.at(in_tensor), wdt_, s_.sd);
  }

  int layer(int l, int x_in) {
    const std::string hf = "model.layers." + std::to_string(l) + ".", tag = "L" + std::to_string(l) + ".";
    std::map<std::string, int> local{{"x", x_in}};
    in_cols_[x_in] = s_.dim;
    for (const Step& st : kLayerSteps) {
      std::vector<int> in;
      for (const char* name : st.in) {
        if (!name) continue;
        if (name[0] == '#') {
          in.push_back(st.type == OpType::RMSNORM ? norm(hf + (name + 1)) : layer_weight(hf + (name + 1), in.at(0), st.width));
        } else {
          in.push_back(local.at(name));
        }
      }
      const int out = b_.activation(tag + st.out, width(st.width));
      in_cols_[out] = width(st.width);
      local[st.out] = out;
      std::vector<int32_t> ia;
      std::vector<float> fa;
      switch (st.attr) {
        case A_NORM: fa = {s_.norm_eps}; break;
        case A_ROPE_Q: ia = {s_.n_heads, s_.head_dim}; fa = {s_.rope_theta}; break;
        case A_ROPE_K: ia = {s_.n_kv_heads, s_.head_dim}; fa = {s_.rope_theta}; break;
        case A_ATTN: ia = {l, s_.n_heads, s_.n_kv_heads, 0}; fa = {s_.rope_theta}; break;
        default: break;
      }
      b_.op(st.type, tag + st.op, in, {out}, ia, fa);
    }
    return local.at(kLayerOutput);
  }

  // norm weights: f32 [1, dim], 1 + N(0, norm_sd)
  int norm(const std::string& name) {
    std::vector<uint8_t> data(static_cast<size_t>(s_.dim) * sizeof(float));
    normal_row(s_.seed, serial_++, 0, 1.0f, s_.norm_sd, reinterpret_cast<float*>(data.data()), s_.dim);
    return b_.weight(name, DType::F32, 1, s_.dim, std::move(data), {});
  }

  // an N(0, sd) matrix, quantized to dt row block by row block
  int matrix(const std::string& name, int64_t rows, int64_t cols, DType dt, float sd) {
    const uint64_t id = serial_++;
    const size_t r = static_cast<size_t>(rows), c = static_cast<size_t>(cols);
    std::vector<uint8_t> data(dt == DType::F32 ? r * c * 4 : dt == DType::Q8 ? r * c : r * c / 2);
    std::vector<uint8_t> scales(dt == DType::F32 ? 0 : (dt == DType::Q8 ? r : r * c / 32) * sizeof(float));
    if (dt == DType::Q4 && cols % 32) throw std::runtime_error("edgelm: q4 needs K % 32 == 0 (" + name + ")");
    constexpr int64_t kRowsPerTask = 64;
    const int64_t tasks = (rows + kRowsPerTask - 1) / kRowsPerTask;
    over_rows(tasks, s_.threads, [&](int64_t task) {
      const int64_t r0 = task * kRowsPerTask, nr = std::min(kRowsPerTask, rows - r0);
      std::vector<float> f(static_cast<size_t>(nr * cols));
      for (int64_t i = 0; i < nr; ++i) normal_row(s_.seed, id, static_cast<uint64_t>(r0 + i), 0.0f, sd, &f[i * cols], cols);
      if (dt == DType::F32) {
        std::memcpy(data.data() + r0 * cols * 4, f.data(), f.size() * 4);
      } else if (dt == DType::Q8) {
        elm_quantize_q8(f.data(), nr, cols, reinterpret_cast<int8_t*>(data.data()) + r0 * cols,
                        reinterpret_cast<float*>(scales.data()) + r0, 1);
      } else {
        elm_quantize_q4(f.data(), nr, cols, data.data() + r0 * cols / 2,
                        reinterpret_cast<float*>(scales.data()) + r0 * (cols / 32), 1);
      }
    });
    return b_.weight(name, dt, rows, cols, std::move(data), std::move(scales));
  }

  const elm_model_spec& s_;
  DType wdt_, edt_;
  ContainerBuilder b_;
  uint64_t serial_ = 0;  // tensor index of the random stream
  std::map<int, int64_t> in_cols_;
};

}  // namespace

void write_random_model(const std::string& path, const elm_model_spec& s) {
  if (s.vocab < 1 || s.dim < 1 || s.hidden < 1 || s.n_layers < 0 || s.n_heads < 1 || s.n_kv_heads < 1 || s.head_dim < 2 ||
      s.head_dim % 2 || s.max_seq < 1 || s.n_heads % s.n_kv_heads)
    throw std::runtime_error("edgelm: bad model shape");
  Synth(s).build(path);
}

}  // namespace edgelm

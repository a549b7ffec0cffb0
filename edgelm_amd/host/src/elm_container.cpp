// Reading an .elm container into a Model. The byte layout is the one edgelm's exporter writes
// (tools/elm.py:207-276) and edgelm's loader reads (model.cpp:67-148); it is declared here once as
// packed records, and every fixed-size record is taken from the file in one copy:
//
//   bytes [0, 128)   ContainerHeader: magic, version, record counts, where the three sections are,
//                    the model config and flags
//   graph section    per tensor: u16 name length, name, TensorRecord; then per op: OpRecord, the
//                    int32 input and output tensor ids, OpAttrs, u16 name length, name
//   tokenizer        edgelm's vocabulary and merges (only its extent is checked against the file:
//                    this build runs token ids and never parses the section)
//   weight blob      the arrays, each 64-byte aligned, at offsets relative to the blob start
#include "edgelm/elm_container.hpp"

#include <cstring>
#include <stdexcept>

#include "edgelm/file_map.hpp"
#include "edgelm/model.hpp"
#include "edgelm_host.h"

namespace edgelm {
namespace {

[[noreturn]] void corrupt(const std::string& what) { throw std::runtime_error("edgelm: malformed .elm file: " + what); }

// Sequential reads from one section, every read checked against the section's end.
class SectionReader {
 public:
  SectionReader(const uint8_t* data, uint64_t len, const char* section) : p_(data), left_(len), section_(section) {}
  template <class Pod>
  Pod pod() {
    Pod v;
    std::memcpy(&v, take(sizeof(Pod)), sizeof(Pod));
    return v;
  }
  std::string name() {
    const uint16_t n = pod<uint16_t>();
    return std::string(reinterpret_cast<const char*>(take(n)), n);
  }
  void ids(uint8_t count, std::vector<int>& out) {
    const uint8_t* p = take(static_cast<size_t>(count) * sizeof(int32_t));
    for (uint8_t i = 0; i < count; ++i) {
      int32_t v;
      std::memcpy(&v, p + i * sizeof(int32_t), sizeof v);
      out.push_back(v);
    }
  }

 private:
  const uint8_t* take(size_t n) {
    if (n > left_) corrupt(std::string("the ") + section_ + " section ends inside a record");
    const uint8_t* p = p_;
    p_ += n;
    left_ -= n;
    return p;
  }
  const uint8_t* p_;
  uint64_t left_;
  const char* section_;
};

bool section_fits(const ContainerHeader::Section& s, size_t file) { return s.off <= file && s.len <= file - s.off; }

}  // namespace

Model Model::load(const std::string& path) {
  Model m;
  auto file = std::make_shared<const FileMap>(path);
  m.file_ = file;
  if (file->size() < sizeof(ContainerHeader)) corrupt(path + " is shorter than the 128-byte header");
  ContainerHeader h;
  std::memcpy(&h, file->base(), sizeof h);
  if (std::memcmp(h.magic, kElmMagic, 4) != 0) corrupt(path + " does not start with ELM1");
  if (h.version != kElmVersion) corrupt("version " + std::to_string(h.version) + " (this reader knows 1)");
  if (!section_fits(h.graph, file->size()) || !section_fits(h.tok, file->size()) || !section_fits(h.blob, file->size()))
    corrupt("a section lies outside the file");

  Config& c = m.cfg;
  c.vocab = static_cast<int>(h.vocab);
  c.dim = static_cast<int>(h.dim);
  c.hidden = static_cast<int>(h.hidden);
  c.n_layers = static_cast<int>(h.n_layers);
  c.n_heads = static_cast<int>(h.n_heads);
  c.n_kv_heads = static_cast<int>(h.n_kv_heads);
  c.head_dim = static_cast<int>(h.head_dim);
  c.max_seq = static_cast<int>(h.max_seq);
  c.rope_theta = h.rope_theta;
  c.norm_eps = h.norm_eps;
  c.bos = static_cast<int>(h.bos);
  c.eos = static_cast<int>(h.eos);
  c.weight_dtype = static_cast<DType>(h.weight_dtype);
  c.tied = (h.flags & kElmFlagTied) != 0;

  const uint8_t* blob = file->base() + h.blob.off;
  SectionReader r(file->base() + h.graph.off, h.graph.len, "graph");
  // every tensor record takes at least its name length and TensorRecord, every op record at least its
  // OpRecord, OpAttrs and name length: counts the section cannot hold are refused before any allocation
  const uint64_t min_tensor = sizeof(uint16_t) + sizeof(TensorRecord);
  const uint64_t min_op = sizeof(OpRecord) + sizeof(OpAttrs) + sizeof(uint16_t);
  if (h.n_tensors > h.graph.len / min_tensor || h.n_ops > (h.graph.len - h.n_tensors * min_tensor) / min_op)
    corrupt(std::to_string(h.n_tensors) + " tensors and " + std::to_string(h.n_ops) + " ops cannot fit a graph section of " +
            std::to_string(h.graph.len) + " bytes");
  m.graph.tensors.resize(h.n_tensors);
  for (Tensor& t : m.graph.tensors) {
    t.name = r.name();
    const TensorRecord rec = r.pod<TensorRecord>();
    t.kind = static_cast<TensorKind>(rec.kind);
    t.dtype = static_cast<DType>(rec.dtype);
    t.rows_sym = static_cast<RowSym>(rec.rows_sym);
    t.rows = rec.rows;
    t.cols = rec.cols;
    t.group = static_cast<int>(rec.group);
    if (!t.is_weight()) continue;
    const bool data_ok = rec.data_off <= h.blob.len && rec.data_len <= h.blob.len - rec.data_off;
    const bool scale_ok = rec.scale_off <= h.blob.len && rec.scale_len <= h.blob.len - rec.scale_off;
    if (!data_ok || !scale_ok) corrupt("weight " + t.name + " lies outside the weight blob");
    t.data = blob + rec.data_off;
    t.data_bytes = rec.data_len;
    if (rec.scale_len) {
      t.scales = reinterpret_cast<const float*>(blob + rec.scale_off);
      t.scale_bytes = rec.scale_len;
    }
  }
  m.graph.ops.resize(h.n_ops);
  const int nt = static_cast<int>(h.n_tensors);
  for (Op& op : m.graph.ops) {
    const OpRecord rec = r.pod<OpRecord>();
    if (rec.type >= static_cast<uint8_t>(OpType::COUNT)) corrupt("op type " + std::to_string(rec.type));
    op.type = static_cast<OpType>(rec.type);
    r.ids(rec.n_in, op.in);
    r.ids(rec.n_out, op.out);
    const OpAttrs at = r.pod<OpAttrs>();
    std::memcpy(op.iattr, at.iattr, sizeof op.iattr);
    std::memcpy(op.fattr, at.fattr, sizeof op.fattr);
    op.name = r.name();
    for (const std::vector<int>* ids : {&op.in, &op.out})
      for (int t : *ids)
        if (t < 0 || t >= nt) corrupt("op " + op.name + " names tensor " + std::to_string(t));
  }
  m.graph.index_io();
  return m;
}

size_t Model::weight_bytes() const {
  size_t total = 0;
  for (const Tensor& t : graph.tensors) total += t.is_weight() ? t.data_bytes + t.scale_bytes : 0;
  return total;
}

size_t Model::file_bytes() const { return file_ ? file_->size() : 0; }

void Model::prefault() const {
  if (!file_) return;
  ::madvise(const_cast<uint8_t*>(file_->base()), file_->size(), MADV_WILLNEED);
  const long page = ::sysconf(_SC_PAGESIZE);
  const size_t step = page > 0 ? static_cast<size_t>(page) : 4096;
  uint8_t acc = 0;
  for (size_t at = 0; at < file_->size(); at += step) acc ^= reinterpret_cast<const volatile uint8_t*>(file_->base())[at];
  (void)acc;
}

void Model::convert_weights(DType target, int threads) {
  if (target == DType::F32) {
    if (cfg.weight_dtype != DType::F32) throw std::runtime_error("edgelm: a quantized model cannot be converted to f32");
    return;
  }
  if (target != DType::Q8 && target != DType::Q4) throw std::runtime_error("edgelm: convert_weights takes q8 or q4");
  for (Tensor& t : graph.tensors) {
    if (!t.is_weight() || t.dtype != DType::F32 || t.rows <= 1) continue;  // norm vectors stay f32
    const bool q8 = target == DType::Q8;
    if (!q8 && t.cols % 32) throw std::runtime_error("edgelm: q4 needs K % 32 == 0 (" + t.name + ")");
    const size_t rows = static_cast<size_t>(t.rows), cols = static_cast<size_t>(t.cols);
    auto data = std::make_shared<std::vector<uint8_t>>(q8 ? rows * cols : rows * cols / 2);
    auto scales = std::make_shared<std::vector<uint8_t>>((q8 ? rows : rows * cols / 32) * sizeof(float));
    const float* w = static_cast<const float*>(t.data);
    float* s = reinterpret_cast<float*>(scales->data());
    const int rc = q8 ? elm_quantize_q8(w, t.rows, t.cols, reinterpret_cast<int8_t*>(data->data()), s, threads)
                      : elm_quantize_q4(w, t.rows, t.cols, data->data(), s, threads);
    if (rc) throw std::runtime_error("edgelm: quantizing " + t.name + " failed");
    t.dtype = target;
    t.group = q8 ? static_cast<int>(t.cols) : 32;
    t.data = data->data();
    t.data_bytes = data->size();
    t.scales = s;
    t.scale_bytes = scales->size();
    converted_.push_back(std::move(data));
    converted_.push_back(std::move(scales));
  }
  cfg.weight_dtype = target;
}

void quantize_q8(const float* w, int64_t n, int64_t k, int8_t* out, float* scales) {
  if (elm_quantize_q8(w, n, k, out, scales, 1)) throw std::runtime_error("edgelm: quantize_q8: bad shape");
}

void quantize_q4(const float* w, int64_t n, int64_t k, uint8_t* out, float* scales) {
  if (elm_quantize_q4(w, n, k, out, scales, 1)) throw std::runtime_error("edgelm: q4 needs K % 32 == 0");
}

void dequantize_row(const Tensor& w, int64_t row, float* out) {
  const int64_t k = w.cols;
  if (w.dtype == DType::F32) {
    std::memcpy(out, static_cast<const float*>(w.data) + row * k, sizeof(float) * static_cast<size_t>(k));
  } else if (w.dtype == DType::Q8) {
    const int8_t* q = static_cast<const int8_t*>(w.data) + row * k;
    for (int64_t i = 0; i < k; ++i) out[i] = static_cast<float>(q[i]) * w.scales[row];
  } else if (w.dtype == DType::Q4) {
    // 16 bytes per 32-group: element j of the group in the low nibble of byte j, element j + 16 in
    // the high nibble, each stored as q + 8
    const uint8_t* q = static_cast<const uint8_t*>(w.data) + row * (k / 2);
    const float* s = w.scales + row * (k / 32);
    for (int64_t e = 0; e < k; ++e) {
      const int64_t g = e / 32, j = e % 32;
      const uint8_t byte = q[g * 16 + (j & 15)];
      const int nib = j < 16 ? (byte & 0x0F) : (byte >> 4);
      out[e] = static_cast<float>(nib - 8) * s[g];
    }
  } else {
    throw std::runtime_error("edgelm: dequantize_row: not a weight dtype");
  }
}

}  // namespace edgelm

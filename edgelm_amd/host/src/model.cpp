// .elm loading: a 128-byte header (config + section offsets), tensor records, op records, the
// tokenizer section (skipped: this build runs token ids) and 64-byte aligned weight blobs
// (reference tools/elm.py:207-276, loader model.cpp:67-148).
#include "edgelm/model.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>

#include "edgelm_host.h"

namespace edgelm {

class Mapping {
 public:
  explicit Mapping(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    EDGELM_CHECK(fd >= 0, "cannot open " + path);
    struct stat st {};
    if (::fstat(fd, &st) == 0) size_ = static_cast<size_t>(st.st_size);
    if (size_ > 0) base_ = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    EDGELM_CHECK(size_ > 0 && base_ != MAP_FAILED, "cannot map " + path);
  }
  ~Mapping() {
    if (base_ && base_ != MAP_FAILED) ::munmap(base_, size_);
  }
  Mapping(const Mapping&) = delete;
  Mapping& operator=(const Mapping&) = delete;
  const uint8_t* data() const { return static_cast<const uint8_t*>(base_); }
  size_t size() const { return size_; }

 private:
  void* base_ = nullptr;
  size_t size_ = 0;
};

namespace {

// Bounds-checked little-endian cursor over one section of the file.
class Cursor {
 public:
  Cursor(const uint8_t* p, size_t n) : p_(p), end_(p + n) {}
  template <class V>
  V take() {
    EDGELM_CHECK(static_cast<size_t>(end_ - p_) >= sizeof(V), "truncated model file");
    V v;
    std::memcpy(&v, p_, sizeof(V));
    p_ += sizeof(V);
    return v;
  }
  std::string text(size_t n) {
    EDGELM_CHECK(static_cast<size_t>(end_ - p_) >= n, "truncated model file");
    std::string s(reinterpret_cast<const char*>(p_), n);
    p_ += n;
    return s;
  }

 private:
  const uint8_t* p_;
  const uint8_t* end_;
};

}  // namespace

Model Model::load(const std::string& path) {
  Model m;
  m.map_ = std::make_shared<Mapping>(path);
  const uint8_t* base = m.map_->data();
  const size_t size = m.map_->size();
  EDGELM_CHECK(size >= 128 && std::memcmp(base, "ELM1", 4) == 0, "not an .elm file: " + path);
  Cursor h(base + 4, 124);
  const uint32_t version = h.take<uint32_t>(), n_tensors = h.take<uint32_t>(), n_ops = h.take<uint32_t>();
  EDGELM_CHECK(version == 1, "unsupported .elm version");
  uint64_t off[6];
  for (uint64_t& o : off) o = h.take<uint64_t>();
  const uint64_t graph_off = off[0], graph_size = off[1], w_off = off[4], w_size = off[5];
  EDGELM_CHECK(graph_off + graph_size <= size && off[2] + off[3] <= size && w_off + w_size <= size,
               "section out of bounds");
  Config& c = m.cfg;
  for (int* v : {&c.vocab, &c.dim, &c.hidden, &c.n_layers, &c.n_heads, &c.n_kv_heads, &c.head_dim, &c.max_seq})
    *v = static_cast<int>(h.take<uint32_t>());
  c.rope_theta = h.take<float>();
  c.norm_eps = h.take<float>();
  c.bos = static_cast<int>(h.take<uint32_t>());
  c.eos = static_cast<int>(h.take<uint32_t>());
  c.weight_dtype = static_cast<DType>(h.take<uint32_t>());
  (void)h.take<uint32_t>();  // group size (repeated per tensor)
  c.tied = (h.take<uint32_t>() & 1) != 0;

  Cursor g(base + graph_off, graph_size);
  const uint8_t* wbase = base + w_off;
  for (uint32_t i = 0; i < n_tensors; ++i) {
    Tensor t;
    t.name = g.text(g.take<uint16_t>());
    t.kind = static_cast<TensorKind>(g.take<uint8_t>());
    t.dtype = static_cast<DType>(g.take<uint8_t>());
    t.rows_sym = static_cast<RowSym>(g.take<uint8_t>());
    (void)g.take<uint8_t>();
    t.rows = g.take<int64_t>();
    t.cols = g.take<int64_t>();
    const uint64_t doff = g.take<uint64_t>(), dbytes = g.take<uint64_t>();
    const uint64_t soff = g.take<uint64_t>(), sbytes = g.take<uint64_t>();
    t.group = static_cast<int>(g.take<uint32_t>());
    if (t.is_weight()) {
      EDGELM_CHECK(doff + dbytes <= w_size && soff + sbytes <= w_size, "weight out of bounds: " + t.name);
      t.data = wbase + doff;
      t.data_bytes = dbytes;
      if (sbytes) {
        t.scales = reinterpret_cast<const float*>(wbase + soff);
        t.scale_bytes = sbytes;
      }
    }
    m.graph.tensors.push_back(std::move(t));
  }
  for (uint32_t i = 0; i < n_ops; ++i) {
    Op op;
    op.type = static_cast<OpType>(g.take<uint8_t>());
    EDGELM_CHECK(op.type < OpType::COUNT, "unknown op type");
    const int ni = g.take<uint8_t>(), no = g.take<uint8_t>();
    (void)g.take<uint8_t>();
    for (int j = 0; j < ni; ++j) op.in.push_back(g.take<int32_t>());
    for (int j = 0; j < no; ++j) op.out.push_back(g.take<int32_t>());
    for (int& a : op.iattr) a = g.take<int32_t>();
    for (float& a : op.fattr) a = g.take<float>();
    op.name = g.text(g.take<uint16_t>());
    for (int t : op.in) EDGELM_CHECK(t >= 0 && t < static_cast<int>(n_tensors), "bad tensor reference");
    for (int t : op.out) EDGELM_CHECK(t >= 0 && t < static_cast<int>(n_tensors), "bad tensor reference");
    m.graph.ops.push_back(std::move(op));
  }
  m.graph.index_io();
  return m;
}

size_t Model::weight_bytes() const {
  size_t n = 0;
  for (const Tensor& t : graph.tensors)
    if (t.is_weight()) n += t.data_bytes + t.scale_bytes;
  return n;
}

void quantize_q8(const float* w, int64_t n, int64_t k, int8_t* out, float* scales) {
  elm_quantize_q8(w, n, k, out, scales, 1);
}

void quantize_q4(const float* w, int64_t n, int64_t k, uint8_t* out, float* scales) {
  EDGELM_CHECK(k % 32 == 0, "q4 needs K % 32 == 0");
  elm_quantize_q4(w, n, k, out, scales, 1);
}

void dequantize_row(const Tensor& w, int64_t row, float* out) {
  const int64_t k = w.cols;
  switch (w.dtype) {
    case DType::F32:
      std::memcpy(out, static_cast<const float*>(w.data) + row * k, sizeof(float) * static_cast<size_t>(k));
      return;
    case DType::Q8: {
      const int8_t* q = static_cast<const int8_t*>(w.data) + row * k;
      const float s = w.scales[row];
      for (int64_t i = 0; i < k; ++i) out[i] = static_cast<float>(q[i]) * s;
      return;
    }
    case DType::Q4: {
      const uint8_t* q = static_cast<const uint8_t*>(w.data) + row * (k / 2);
      const float* s = w.scales + row * (k / 32);
      for (int64_t g = 0; g < k / 32; ++g)
        for (int i = 0; i < 16; ++i) {
          out[g * 32 + i] = static_cast<float>(static_cast<int>(q[g * 16 + i] & 0x0F) - 8) * s[g];
          out[g * 32 + 16 + i] = static_cast<float>(static_cast<int>(q[g * 16 + i] >> 4) - 8) * s[g];
        }
      return;
    }
    default:
      EDGELM_CHECK(false, "dequantize_row: bad dtype");
  }
}

}  // namespace edgelm

// .elm model loader (format of the reference's tools/elm.py:1-9, 207-276; C++ loader model.cpp:67-148):
// the file is memory-mapped and weight tensors point into the mapping.
#pragma once
#include <memory>
#include <string>
#include <vector>

#include "edgelm/graph.hpp"

namespace edgelm {

struct Config {
  int vocab = 0, dim = 0, hidden = 0, n_layers = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0, max_seq = 0;
  float rope_theta = 10000.f, norm_eps = 1e-5f;
  int bos = 0, eos = 0;
  DType weight_dtype = DType::F32;
  bool tied = false;
};

class Mapping;

class Model {
 public:
  static Model load(const std::string& path);
  size_t weight_bytes() const;

  Config cfg;
  Graph graph;

 private:
  std::shared_ptr<Mapping> map_;
};

// edgelm's quantizers (model.cpp:150-190) and row dequantization (model.cpp:192-218).
void quantize_q8(const float* w, int64_t n, int64_t k, int8_t* out, float* scales);
void quantize_q4(const float* w, int64_t n, int64_t k, uint8_t* out, float* scales);
void dequantize_row(const Tensor& w, int64_t row, float* out);

}  // namespace edgelm

// A model as the runtime sees it: the config, the (unfused) graph and the weight arrays of an .elm
// container (the file format of edgelm's exporter, tools/elm.py:207-276; edgelm's Model is
// include/edgelm/model.hpp:29-53). Weights point into a read-only mapping of the file, or into
// buffers the model owns after convert_weights().
#pragma once
#include <cstdint>
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

class FileMap;

class Model {
 public:
  static Model load(const std::string& path);

  // Quantize every f32 weight matrix (more than one row) to q8 or q4 in memory, as edgelm's
  // Model::convert_weights does at load for `--dtype` (model.cpp:220-251, main.cpp:53-60): the same
  // quantizers, byte for byte; norm vectors stay f32. F32 keeps an f32 file as it is and refuses a
  // quantized one. Runs the rows over `threads` host threads.
  void convert_weights(DType target, int threads = 1);
  // Read every page of the mapping once, so the first forward does not take the page faults
  // (edgelm's Model::prefault, model.cpp:260-266).
  void prefault() const;
  size_t weight_bytes() const;  // data + scales of every weight
  size_t file_bytes() const;

  // Device image: every q8 / q4 weight in the repacked layout the hip delegate keeps in HBM
  // (elmh_repack_host), in one file, so that a later session uploads each weight as it will lie in
  // HBM. The image records a digest of the model (its config, tensor table and every byte of every
  // weight's data and scales);
  // attach_device_image maps an image and points the weights at it, or returns false (and changes
  // nothing) when the file is missing or was written for other weights. Returns the weights written.
  int write_device_image(const std::string& path, int threads = 1) const;
  bool attach_device_image(const std::string& path);
  uint64_t digest() const;

  Config cfg;
  Graph graph;

 private:
  std::shared_ptr<const FileMap> file_;
  std::shared_ptr<const FileMap> image_;  // an attached device image
  std::vector<std::shared_ptr<std::vector<uint8_t>>> converted_;  // arrays made by convert_weights
};

// edgelm's quantizers (model.cpp:150-190) and row dequantization (model.cpp:192-218).
void quantize_q8(const float* w, int64_t n, int64_t k, int8_t* out, float* scales);
void quantize_q4(const float* w, int64_t n, int64_t k, uint8_t* out, float* scales);
void dequantize_row(const Tensor& w, int64_t row, float* out);

}  // namespace edgelm

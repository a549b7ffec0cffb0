// Graph IR of the edgelm runtime, restated for this build: the enum values and struct members are
// the ones edgelm's .elm files and backends use (reference include/edgelm/graph.hpp:17-64), so a
// backend written against this header compiles against edgelm's unchanged.
#pragma once
#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace edgelm {

#define EDGELM_CHECK(cond, msg)                                                                  \
  do {                                                                                           \
    if (!(cond)) throw std::runtime_error(std::string("edgelm: ") + (msg) + " [" #cond "]");     \
  } while (0)

enum class DType : uint8_t { F32 = 0, Q8 = 1, Q4 = 2, I32 = 3 };
enum class TensorKind : uint8_t { Weight = 0, Activation = 1, Input = 2, Output = 3 };
enum class RowSym : uint8_t { Const = 0, T = 1, L = 2 };  // fixed rows, tokens this step, logit rows

enum class OpType : uint8_t {
  EMBED = 0, RMSNORM, MATMUL, ROPE, ATTENTION, ADD, SILU, MUL, LAST_ROWS,
  MATMUL_N,    // x . W_i^T for several weights sharing x (fused QKV)
  FFN_SWIGLU,  // silu(x . Wg^T) * (x . Wu^T)
  MATMUL_ADD,  // r + x . W^T
  COUNT
};

const char* op_name(OpType t);
const char* dtype_name(DType d);

struct Tensor {
  std::string name;
  TensorKind kind = TensorKind::Activation;
  DType dtype = DType::F32;
  RowSym rows_sym = RowSym::Const;
  int64_t rows = 0, cols = 0;
  const void* data = nullptr;     // weights: into the mapped file (or owned conversion buffers)
  const float* scales = nullptr;  // q8: [rows]; q4: [rows * cols / 32]
  size_t data_bytes = 0, scale_bytes = 0;
  int group = 0;
  // Not in edgelm's Tensor: the weight in a device's repacked layout, from a device image attached to
  // the model (Model::attach_device_image), or null. Code that must also compile against edgelm's
  // header tests EDGELM_TENSOR_DEVICE_IMAGE.
  const void* image = nullptr;
  const float* image_scales = nullptr;
  bool is_weight() const { return kind == TensorKind::Weight; }
};
#define EDGELM_TENSOR_DEVICE_IMAGE 1

struct Op {
  OpType type = OpType::COUNT;
  std::string name;
  std::vector<int> in, out;
  int iattr[4] = {0, 0, 0, 0};  // ROPE: n_heads, head_dim | ATTENTION: layer, n_heads, n_kv, fused_rope
  float fattr[2] = {0, 0};      // RMSNORM: eps | ROPE / ATTENTION: theta
};

struct Graph {
  std::vector<Tensor> tensors;
  std::vector<Op> ops;
  int input = -1;   // token ids
  int output = -1;  // logits
  void index_io();
  std::vector<std::vector<int>> consumers() const;
  std::string summary() const;
};

}  // namespace edgelm

// The fixed-size records of the .elm container, little-endian and packed exactly as edgelm's exporter
// writes them (tools/elm.py:207-276: struct formats "<III", "<QQQQQQ", "<8I", "<ffII", "<III" for the
// header, "<BBBBqqQQQQI" per tensor, "<BBBB" + "<4i2f" per op). Shared by the reader (Model::load)
// and the writer of synthetic models.
#pragma once
#include <cstdint>

namespace edgelm {

constexpr char kElmMagic[4] = {'E', 'L', 'M', '1'};
constexpr uint32_t kElmVersion = 1;
constexpr uint32_t kElmFlagTied = 1;  // header flags bit 0: the LM head is the embedding
constexpr uint64_t kElmAlign = 64;     // weight arrays (and the blob itself) start at multiples of 64

#pragma pack(push, 1)
struct ContainerHeader {
  char magic[4];
  uint32_t version, n_tensors, n_ops;
  struct Section {
    uint64_t off, len;  // absolute file offset and length
  } graph, tok, blob;
  uint32_t vocab, dim, hidden, n_layers, n_heads, n_kv_heads, head_dim, max_seq;
  float rope_theta, norm_eps;
  uint32_t bos, eos;
  uint32_t weight_dtype, group, flags;
  uint8_t reserved[4];
};

struct TensorRecord {  // follows the tensor's u16-prefixed name
  uint8_t kind, dtype, rows_sym, reserved;
  int64_t rows, cols;
  uint64_t data_off, data_len, scale_off, scale_len;  // relative to the weight blob
  uint32_t group;
};

struct OpRecord {  // then n_in + n_out int32 tensor ids, OpAttrs, the u16-prefixed name
  uint8_t type, n_in, n_out, reserved;
};

struct OpAttrs {
  int32_t iattr[4];
  float fattr[2];
};
#pragma pack(pop)

static_assert(sizeof(ContainerHeader) == 128, "header is 128 bytes");
static_assert(sizeof(TensorRecord) == 56, "tensor record is <BBBBqqQQQQI>");
static_assert(sizeof(OpRecord) == 4 && sizeof(OpAttrs) == 24, "op record is <BBBB> ... <4i2f>");

}  // namespace edgelm

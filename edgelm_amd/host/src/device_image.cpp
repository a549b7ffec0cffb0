// Device image of a model: its q8 / q4 weights in the repacked layout the hip delegate keeps in HBM
// (include/elmh.h: elmh_weight_layout, elmh_repack_host), cached in one file so that a later session
// uploads every weight as it will lie in HBM, with no export-layout staging and no repack launch per
// weight. The load path it shortens is edgelm's model.cpp:94-116 (weights mapped from the .elm file).
//
//   bytes [0, 64)       ImageHeader: magic, version, entry count, the model digest, where the table
//                       and the arrays are, the file size
//   table               ImageEntry per weight: name, dtype, tile height, shape, where its repacked
//                       data and scales are
//   arrays              each 256-byte aligned
//
// The digest covers the config, the tensor table and every byte of every weight's data and scales
// (hashed in parallel, each 8-byte word through a full 64-bit finalizer so that any changed bit moves
// the whole hash), so an image written for other weights is refused.
#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <thread>
#include <unordered_map>

#include "edgelm/file_map.hpp"
#include "edgelm/model.hpp"
#include "elmh.h"

namespace edgelm {
namespace {

constexpr char kImageMagic[8] = {'E', 'L', 'M', 'H', 'I', 'M', 'G', '1'};
constexpr uint32_t kImageVersion = 1;
constexpr uint64_t kImageAlign = 256;

struct ImageHeader {
  char magic[8];
  uint32_t version;
  uint32_t n_entries;
  uint64_t digest;
  uint64_t table_offset;
  uint64_t data_offset;
  uint64_t file_bytes;
  uint8_t reserved[16];
};
static_assert(sizeof(ImageHeader) == 64, "image header is 64 bytes");

struct ImageEntry {
  char name[128];  // NUL-terminated
  uint32_t dtype, H;
  int64_t rows, cols;
  uint64_t data_offset, data_bytes, scale_offset, scale_bytes;
  uint64_t reserved;
};
static_assert(sizeof(ImageEntry) == 192, "image entry is 192 bytes");

uint64_t align_up(uint64_t v) { return (v + kImageAlign - 1) / kImageAlign * kImageAlign; }

// 64-bit hash of byte strings fed in order. Each 8-byte word goes through murmur3's fmix64 finalizer
// before it is folded in, so a change in any bit of any word changes every bit of the result with
// probability 1/2; four lanes take the words in turn so the folds do not form one dependent chain.
class Digest {
 public:
  static uint64_t fmix(uint64_t x) {
    x ^= x >> 33;
    x *= 0xff51afd7ed558ccdull;
    x ^= x >> 33;
    x *= 0xc4ceb9fe1a85ec53ull;
    return x ^ (x >> 33);
  }
  void bytes(const void* p, size_t n) {
    const uint8_t* b = static_cast<const uint8_t*>(p);
    uint64_t lane[4] = {h_, h_ ^ 0x9e3779b97f4a7c15ull, h_ ^ 0xbf58476d1ce4e5b9ull, h_ ^ 0x94d049bb133111ebull};
    size_t i = 0;
    for (; i + 32 <= n; i += 32)
      for (int l = 0; l < 4; ++l) {
        uint64_t w;
        std::memcpy(&w, b + i + 8 * l, 8);
        lane[l] = (lane[l] ^ fmix(w)) * 0x100000001b3ull;
      }
    uint64_t tail = n;  // the length, then the bytes past the last whole 32
    for (; i < n; ++i) tail = (tail ^ b[i]) * 0x100000001b3ull;
    h_ = fmix(fmix(fmix(fmix(lane[0]) ^ lane[1]) ^ lane[2]) ^ lane[3]) ^ fmix(tail);
  }
  template <class Pod>
  void pod(const Pod& v) {
    bytes(&v, sizeof v);
  }
  uint64_t value() const { return h_; }

 private:
  uint64_t h_ = 0xcbf29ce484222325ull;
};

// Digest of one array: 1 MiB pieces hashed on `threads` host threads, their hashes folded in order.
uint64_t digest_array(const void* p, size_t n, int threads) {
  constexpr size_t kPiece = size_t(1) << 20;
  const size_t pieces = (n + kPiece - 1) / kPiece;
  std::vector<uint64_t> part(pieces);
  std::atomic<size_t> next{0};
  auto work = [&] {
    for (size_t i; (i = next.fetch_add(1)) < pieces;) {
      Digest d;
      d.bytes(static_cast<const uint8_t*>(p) + i * kPiece, std::min(kPiece, n - i * kPiece));
      part[i] = d.value();
    }
  };
  std::vector<std::thread> pool;
  for (int k = 1; k < std::min<int>(threads, static_cast<int>(pieces)); ++k) pool.emplace_back(work);
  work();
  for (std::thread& th : pool) th.join();
  Digest all;
  all.pod(n);
  if (!part.empty()) all.bytes(part.data(), part.size() * sizeof(uint64_t));
  return all.value();
}

// Host threads for hashing a model's weights.
int digest_threads() { return static_cast<int>(std::clamp(std::thread::hardware_concurrency(), 1u, 8u)); }

// The weights an image holds: q8 / q4 weights whose layout libelmh accepts.
bool imageable(const Tensor& t) {
  if (!t.is_weight() || (t.dtype != DType::Q8 && t.dtype != DType::Q4) || !t.data || !t.scales) return false;
  if (t.name.size() >= sizeof(ImageEntry::name)) return false;
  return elmh_weight_layout(static_cast<int>(t.dtype), t.rows, t.cols, nullptr, nullptr, nullptr) == ELMH_OK;
}

}  // namespace

uint64_t Model::digest() const {
  const int threads = digest_threads();
  Digest d;
  d.pod(cfg.vocab), d.pod(cfg.dim), d.pod(cfg.hidden), d.pod(cfg.n_layers), d.pod(cfg.n_heads);
  d.pod(cfg.n_kv_heads), d.pod(cfg.head_dim), d.pod(cfg.max_seq), d.pod(cfg.rope_theta), d.pod(cfg.norm_eps);
  for (const Tensor& t : graph.tensors) {
    d.bytes(t.name.data(), t.name.size());
    d.pod(t.kind), d.pod(t.dtype), d.pod(t.rows), d.pod(t.cols), d.pod(t.data_bytes), d.pod(t.scale_bytes);
    if (!t.is_weight()) continue;
    if (t.scales) d.pod(digest_array(t.scales, t.scale_bytes, threads));
    if (t.data) d.pod(digest_array(t.data, t.data_bytes, threads));
  }
  return d.value();
}

int Model::write_device_image(const std::string& path, int threads) const {
  std::vector<const Tensor*> ws;
  for (const Tensor& t : graph.tensors)
    if (imageable(t)) ws.push_back(&t);
  std::vector<ImageEntry> table(ws.size());
  uint64_t at = align_up(sizeof(ImageHeader) + table.size() * sizeof(ImageEntry));
  const uint64_t data_offset = at;
  for (size_t i = 0; i < ws.size(); ++i) {
    const Tensor& t = *ws[i];
    ImageEntry& e = table[i];
    std::memset(&e, 0, sizeof e);
    std::memcpy(e.name, t.name.data(), t.name.size());
    int H = 0;
    size_t db = 0, sb = 0;
    elmh_weight_layout(static_cast<int>(t.dtype), t.rows, t.cols, &H, &db, &sb);
    e.dtype = static_cast<uint32_t>(t.dtype);
    e.H = static_cast<uint32_t>(H);
    e.rows = t.rows;
    e.cols = t.cols;
    e.data_offset = at;
    e.data_bytes = db;
    at = align_up(at + db);
    e.scale_offset = at;
    e.scale_bytes = sb;
    at = align_up(at + sb);
  }
  ImageHeader h;
  std::memset(&h, 0, sizeof h);
  std::memcpy(h.magic, kImageMagic, sizeof kImageMagic);
  h.version = kImageVersion;
  h.n_entries = static_cast<uint32_t>(table.size());
  h.digest = digest();
  h.table_offset = sizeof(ImageHeader);
  h.data_offset = data_offset;
  h.file_bytes = at;

  const std::string tmp = path + ".tmp";
  FILE* f = std::fopen(tmp.c_str(), "wb");
  if (!f) throw std::runtime_error("edgelm: cannot write device image " + tmp);
  bool ok = std::fwrite(&h, sizeof h, 1, f) == 1 &&
            (table.empty() || std::fwrite(table.data(), sizeof(ImageEntry), table.size(), f) == table.size());
  // the arrays: each weight repacked in memory by one of the workers, written at its offset in turn
  std::atomic<size_t> next{0};
  std::vector<std::vector<uint8_t>> bufs(ws.size());
  std::atomic<bool> failed{false};
  auto work = [&]() {
    for (size_t i; (i = next.fetch_add(1)) < ws.size();) {
      const Tensor& t = *ws[i];
      std::vector<uint8_t>& b = bufs[i];
      b.assign(table[i].data_bytes + table[i].scale_bytes, 0);
      if (elmh_repack_host(static_cast<int>(t.dtype), t.rows, t.cols, t.data, t.scales, b.data(),
                           reinterpret_cast<float*>(b.data() + table[i].data_bytes)) != ELMH_OK)
        failed = true;
    }
  };
  std::vector<std::thread> pool;
  for (int k = 1; k < std::max(threads, 1); ++k) pool.emplace_back(work);
  work();
  for (std::thread& th : pool) th.join();
  ok = ok && !failed;
  static const uint8_t zeros[kImageAlign] = {};
  uint64_t pos = sizeof h + table.size() * sizeof(ImageEntry);
  auto pad_to = [&](uint64_t target) {
    while (ok && pos < target) {
      const size_t n = static_cast<size_t>(std::min<uint64_t>(target - pos, kImageAlign));
      ok = std::fwrite(zeros, 1, n, f) == n;
      pos += n;
    }
  };
  for (size_t i = 0; ok && i < ws.size(); ++i) {
    const ImageEntry& e = table[i];
    pad_to(e.data_offset);
    ok = ok && std::fwrite(bufs[i].data(), 1, e.data_bytes, f) == e.data_bytes;
    pos += e.data_bytes;
    pad_to(e.scale_offset);
    ok = ok && std::fwrite(bufs[i].data() + e.data_bytes, 1, e.scale_bytes, f) == e.scale_bytes;
    pos += e.scale_bytes;
    std::vector<uint8_t>().swap(bufs[i]);
  }
  pad_to(h.file_bytes);
  ok = std::fclose(f) == 0 && ok;
  if (!ok || std::rename(tmp.c_str(), path.c_str()) != 0) {
    std::remove(tmp.c_str());
    throw std::runtime_error("edgelm: writing device image " + path + " failed");
  }
  return static_cast<int>(ws.size());
}

bool Model::attach_device_image(const std::string& path) {
  if (::access(path.c_str(), R_OK) != 0) return false;
  auto map = std::make_shared<const FileMap>(path);
  if (map->size() < sizeof(ImageHeader)) return false;
  ImageHeader h;
  std::memcpy(&h, map->base(), sizeof h);
  // range checks as `offset <= size && length <= size - offset`, which cannot wrap
  auto fits = [&](uint64_t off, uint64_t len) { return off <= map->size() && len <= map->size() - off; };
  if (std::memcmp(h.magic, kImageMagic, sizeof kImageMagic) != 0 || h.version != kImageVersion ||
      h.file_bytes != map->size() || h.table_offset != sizeof(ImageHeader) ||
      !fits(h.table_offset, uint64_t(h.n_entries) * sizeof(ImageEntry)) || h.digest != digest())
    return false;
  std::unordered_map<std::string, Tensor*> by_name;
  for (Tensor& t : graph.tensors)
    if (imageable(t)) by_name.emplace(t.name, &t);
  std::vector<std::pair<Tensor*, const ImageEntry*>> hits;
  for (uint32_t i = 0; i < h.n_entries; ++i) {
    const ImageEntry* e = reinterpret_cast<const ImageEntry*>(map->base() + h.table_offset) + i;
    if (std::memchr(e->name, 0, sizeof e->name) == nullptr) return false;
    const auto it = by_name.find(e->name);
    if (it == by_name.end()) return false;
    const Tensor& t = *it->second;
    int H = 0;
    size_t db = 0, sb = 0;
    elmh_weight_layout(static_cast<int>(t.dtype), t.rows, t.cols, &H, &db, &sb);
    if (e->dtype != static_cast<uint32_t>(t.dtype) || e->rows != t.rows || e->cols != t.cols ||
        e->H != static_cast<uint32_t>(H) || e->data_bytes != db || e->scale_bytes != sb ||
        e->data_offset % kImageAlign || e->scale_offset % kImageAlign || !fits(e->data_offset, db) ||
        !fits(e->scale_offset, sb))
      return false;
    hits.emplace_back(it->second, e);
  }
  if (hits.size() != by_name.size()) return false;  // an image covers every weight or none
  for (auto& [t, e] : hits) {
    t->image = map->base() + e->data_offset;
    t->image_scales = reinterpret_cast<const float*>(map->base() + e->scale_offset);
  }
  image_ = std::move(map);
  return true;
}

}  // namespace edgelm

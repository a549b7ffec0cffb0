// Load-time weight quantizers, byte-identical to edgelm's quantize_q8 / quantize_q4 (model.cpp:150-190),
// with the rows split over host threads.
#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

#include "edgelm_host.h"

namespace {

// Nearest integer, halves away from zero (edgelm's round_away, model.cpp:63), clamped to [lo, hi] as
// min(hi, max(lo, r)).
inline float level(float v, float lo, float hi) {
  const float r = std::copysign(std::floor(std::fabs(v) + 0.5f), v);
  return std::min(hi, std::max(lo, r));
}

// What a row or group is divided by: its scale, or 1 when the scale is 0 (all-zero data).
inline float divisor(float scale) { return scale == 0.f ? 1.f : scale; }

// q8 (model.cpp:150-163): one scale per row, the row's largest magnitude / 127; levels in [-127, 127].
void q8_rows(const float* w, int64_t r0, int64_t r1, int64_t k, int8_t* out, float* scales) {
  for (int64_t r = r0; r < r1; ++r) {
    const float* src = w + r * k;
    float amax = 0.f;
    for (int64_t i = 0; i < k; ++i) amax = std::max(amax, std::fabs(src[i]));
    scales[r] = amax / 127.0f;
    const float div = divisor(scales[r]);
    std::transform(src, src + k, out + r * k,
                   [div](float v) { return static_cast<int8_t>(level(v / div, -127.f, 127.f)); });
  }
}

// Index of the first element of largest magnitude in x[0, n) (numpy argmax's tie rule).
int first_peak(const float* x, int n) {
  int best = 0;
  for (int i = 1; i < n; ++i)
    if (std::fabs(x[i]) > std::fabs(x[best])) best = i;
  return best;
}

// q4 (model.cpp:165-190): per 32-element group, scale = (signed element of largest magnitude) / -8, levels
// in [-8, 7] stored as level + 8; byte j of the group's 16 holds element j in its low nibble and element
// j + 16 in its high nibble.
void q4_rows(const float* w, int64_t r0, int64_t r1, int64_t k, uint8_t* out, float* scales) {
  constexpr int G = 32, H = G / 2;
  const int64_t groups = k / G;
  for (int64_t r = r0; r < r1; ++r)
    for (int64_t g = 0; g < groups; ++g) {
      const float* src = w + r * k + g * G;
      const float d = src[first_peak(src, G)] / -8.0f;
      scales[r * groups + g] = d;
      const float div = divisor(d);
      auto nibble = [div](float v) { return static_cast<uint8_t>(level(v / div, -8.f, 7.f) + 8); };
      uint8_t* dst = out + r * (k / 2) + g * H;
      for (int j = 0; j < H; ++j) dst[j] = static_cast<uint8_t>(nibble(src[j]) | (nibble(src[j + H]) << 4));
    }
}

template <class F>
void split_rows(int64_t n, int threads, F&& f) {
  threads = std::max(1, std::min<int>(threads, static_cast<int>(std::min<int64_t>(n, 256))));
  if (threads == 1) return f(0, n);
  std::vector<std::thread> ts;
  const int64_t per = (n + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    const int64_t a = t * per, b = std::min(n, a + per);
    if (a < b) ts.emplace_back([=, &f] { f(a, b); });
  }
  for (auto& t : ts) t.join();
}

}  // namespace

extern "C" int elm_quantize_q8(const float* w, int64_t n, int64_t k, int8_t* out, float* scales, int threads) {
  if (n < 0 || k < 1 || (n && (!w || !out || !scales))) return -1;
  split_rows(n, threads, [&](int64_t a, int64_t b) { q8_rows(w, a, b, k, out, scales); });
  return 0;
}

// edgelm's quantize_q4 refuses K % 32 != 0 through EDGELM_CHECK (model.cpp:165-167); so does this one,
// before writing anything.
extern "C" int elm_quantize_q4(const float* w, int64_t n, int64_t k, uint8_t* out, float* scales, int threads) {
  if (n < 0 || k < 32 || k % 32 || (n && (!w || !out || !scales))) return -1;
  split_rows(n, threads, [&](int64_t a, int64_t b) { q4_rows(w, a, b, k, out, scales); });
  return 0;
}

// Load-time weight quantizers (edgelm model.cpp:150-190), split over host threads by rows.
#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

#include "edgelm_host.h"

namespace {

inline float round_away(float v) { return std::copysign(std::floor(std::fabs(v) + 0.5f), v); }  // model.cpp:63

void q8_rows(const float* w, int64_t r0, int64_t r1, int64_t k, int8_t* out, float* scales) {
  for (int64_t r = r0; r < r1; ++r) {
    const float* row = w + r * k;
    float amax = 0.f;
    for (int64_t i = 0; i < k; ++i) amax = std::max(amax, std::fabs(row[i]));
    const float s = amax / 127.0f;
    const float safe = s == 0.f ? 1.f : s;
    scales[r] = s;
    for (int64_t i = 0; i < k; ++i)
      out[r * k + i] = static_cast<int8_t>(std::min(127.f, std::max(-127.f, round_away(row[i] / safe))));
  }
}

void q4_rows(const float* w, int64_t r0, int64_t r1, int64_t k, uint8_t* out, float* scales) {
  constexpr int G = 32;
  for (int64_t r = r0; r < r1; ++r)
    for (int64_t g = 0; g < k / G; ++g) {
      const float* x = w + r * k + g * G;
      int best = 0;  // first element of largest magnitude
      float amax = std::fabs(x[0]);
      for (int i = 1; i < G; ++i)
        if (std::fabs(x[i]) > amax) {
          amax = std::fabs(x[i]);
          best = i;
        }
      const float d = x[best] / -8.0f;
      const float safe = d == 0.f ? 1.f : d;
      scales[r * (k / G) + g] = d;
      uint8_t* o = out + r * (k / 2) + g * (G / 2);
      auto q = [&](float v) { return static_cast<uint8_t>(std::min(7.f, std::max(-8.f, round_away(v / safe))) + 8); };
      for (int i = 0; i < G / 2; ++i) o[i] = static_cast<uint8_t>(q(x[i]) | (q(x[i + G / 2]) << 4));
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

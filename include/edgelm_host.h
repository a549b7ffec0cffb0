/*
 * C API of the edgelm_amd host library (libedgelm_host.so): the C++17 restatement of the edgelm
 * host pieces the hot path needs around it, for callers that are not C++ (tests, bench.py).
 */
#ifndef EDGELM_HOST_H
#define EDGELM_HOST_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Load-time quantizers, bit-identical to edgelm's quantize_q8 (model.cpp:150-163) and
 * quantize_q4 (model.cpp:165-190); rows are split over `threads` host threads. */
void elm_quantize_q8(const float* w, int64_t n, int64_t k, int8_t* out, float* scales, int threads);
void elm_quantize_q4(const float* w, int64_t n, int64_t k, uint8_t* out, float* scales, int threads);

#ifdef __cplusplus
}
#endif
#endif

// Loads straight into LDS (global_load_lds) and the waits and barriers that go with them, for the
// kernels of both device sources.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace elmh {

typedef __attribute__((address_space(3))) unsigned char* LdsBytes;

// One global_load_lds of 16 (or 4) bytes per active lane into LDS at dst + 16 (4) * lane (dst is
// wave-uniform: it goes to M0). Written as asm so that the compiler's wait-count pass does not
// track it (it would drain every in-flight load before each LDS read); the kernel waits for these
// loads itself (wait_vm) and drains them all before its LDS is reused or released. M0 is a
// register the compiler reserves and does not save around asm; the kernels that use these (the
// streaming GEMV, the GEMM and the decode attention) make no other use of it (their code
// references M0 only inside these statements), so the write disturbs nothing.
__device__ __forceinline__ void dma16(const void* src, unsigned char* dst) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(LdsBytes)dst);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory");
}
__device__ __forceinline__ void dma4(const void* src, unsigned char* dst) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(LdsBytes)dst);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(m0) : "memory");
}
// The same from a wave-uniform base (scalar registers) plus a 32-bit byte offset per lane: a loop
// that walks the base keeps the per-lane address arithmetic out of its body. The base must be the
// same in every lane; it is read from the first active one.
__device__ __forceinline__ uint64_t uniform_addr(const void* p) {
  const uint64_t v = (uint64_t)(size_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (uint64_t)hi << 32 | lo;
}
// dst: the LDS byte address (wave-uniform) the lanes' data go to.
__device__ __forceinline__ void dma16s(const void* base, uint32_t off, unsigned dst) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(dst);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(uniform_addr(base)), "s"(m0) : "memory");
}
__device__ __forceinline__ void dma4s(const void* base, uint32_t off, unsigned dst) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(dst);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(uniform_addr(base)), "s"(m0) : "memory");
}

// s_waitcnt vmcnt(N) only (gfx9 encoding: vmcnt[3:0] | expcnt 7 | lgkmcnt 15 | vmcnt[5:4] << 14)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// workgroup barrier for LDS data: this wave's LDS accesses complete (lgkmcnt(0)) before it, and
// the compiler keeps memory accesses on their side of it, but loads from memory (vmcnt) and
// copies into LDS stay in flight
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt 63 and expcnt 7: no wait
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace elmh

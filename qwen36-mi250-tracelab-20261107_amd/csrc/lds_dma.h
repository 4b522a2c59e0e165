// Helpers for kernels that stage operands with global -> LDS DMA loads
// (global_load_lds_dwordx4) on gfx950.
//
// While DMA loads are in flight the compiler treats the vmcnt counter as unordered and
// waits for all of them before any LDS read it issues, which would drain every prefetch.
// Kernels that prefetch with DMA therefore read their MFMA fragments through the inline
// asm below, wait for fragment reads with an explicit lgkmcnt wait, and fence their ring
// stages with explicit vmcnt waits (wait_loads) whose counts follow their own issue order.
#pragma once

#include <stdint.h>

#include "moe_common.h"

namespace moe {

typedef unsigned u32x4v __attribute__((ext_vector_type(4)));

// 16 bytes from LDS byte address addr + OFF (completes at lds_frags_ready).
template <int OFF>
__device__ __forceinline__ u32x4v lds_read_frag(uint32_t addr) {
  u32x4v r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
__device__ __forceinline__ void lds_frags_ready() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}
// Ties a fragment to the wait above: its users cannot move before it.
__device__ __forceinline__ void after_wait(u32x4v& v) { asm volatile("" : "+v"(v)); }

__device__ __forceinline__ f32x4_t mfma_frag(u32x4v a, u32x4v b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Wait until at most n (0..24) of this wave's DMA loads are still in flight.
__device__ __forceinline__ void wait_loads(int n) {
  switch (n) {
#define W(N)                                              \
  case N:                                                 \
    asm volatile("s_waitcnt vmcnt(" #N ")" ::: "memory"); \
    break;
    W(24) W(23) W(22) W(21) W(20) W(19) W(18) W(17) W(16) W(15) W(14) W(13)
    W(12) W(11) W(10) W(9) W(8) W(7) W(6) W(5) W(4) W(3) W(2) W(1)
#undef W
    default:
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

// One global -> LDS DMA load of a wave: lane l's 16 bytes at g go to lds + 16 l (lds is
// wave-uniform). A plain function, so that the builtin's operands are checked once and not
// per template instantiation of its callers (where the host pass would drop the kernel).
__device__ __forceinline__ void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}

// The LDS byte address of a __shared__ / dynamic-shared pointer.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  typedef __attribute__((address_space(3))) const char lds_char;
  return (uint32_t)(uintptr_t)(lds_char*)p;
}

}  // namespace moe

// Direct-to-LDS streaming helpers shared by the skinny-M kernels
// (gemm_decode.hip, gemm_stream.hip): each wave streams its own items through
// private LDS regions and waits on its own vector-memory counter.
#pragma once

#include <type_traits>
#include <utility>

#include "gemm_core.h"

#pragma clang diagnostic ignored "-Winline-asm"

namespace dsl {

namespace dec {

DSL_DEV uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
// 16 bytes per lane from `src` into LDS at m0 + lane*16 (the s_nop covers
// the m0 -> LDS-DMA wait state the compiler cannot see inside the asm).
DSL_DEV void dma16(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src),
               "s"(lds)
               : "memory", "m0");
}
// 4 bytes per lane from `src` into LDS at m0 + lane*4.
DSL_DEV void dma4(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src),
               "s"(lds)
               : "memory", "m0");
}
// Same as dma16, with the non-temporal hint (streamed data, read once).
DSL_DEV void dma16_nt(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src),
               "s"(lds)
               : "memory", "m0");
}
// s_waitcnt vmcnt(N) / lgkmcnt(0) as compiler memory barriers: LDS reads of
// a region may not move above the wait for its loads, nor DMA into a region
// above the wait for its reads.
template <int N>
DSL_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
DSL_DEV void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// f(integral_constant<int, K>) for K = B .. E-1, in order
template <int B, int E, class F>
DSL_DEV void static_for(F &&f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

}  // namespace dec

}  // namespace dsl

// Device helpers shared by the streamed grouped GEMMs (gemm_stream.hip, gemm_wide.hip): global
// stores as inline assembly, LDS-DMA with a wavefront-uniform base, and a loop over positions
// whose index is a compile-time constant.
#pragma once
#include <type_traits>

#include "device.hpp"

namespace moe {

// Global stores written as inline assembly. With stores pending among its loads the compiler
// treats the vector-memory counter as unordered and waits for every load, so a kernel whose
// register rings must stay in flight across its epilogue hides its stores from the count (a
// store the count does not include can only make a later wait longer, never shorter). Each ends
// with wait states of its own: the compiler's hazard checks do not see an assembly store, and it
// rewrote a store's data registers with the next instruction before the store had read them
// (measured: the first 8 bytes of 16-byte stores came out wrong without the s_nop).
typedef unsigned int str_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void str_st16(void *p, uint4 v) {
  const u32x4 w = {v.x, v.y, v.z, v.w};
  asm volatile("global_store_dwordx4 %0, %1, off\n\ts_nop 4" ::"v"(p), "v"(w) : "memory");
}
__device__ __forceinline__ void str_st8(void *p, uint2 v) {
  const str_u32x2 w = {v.x, v.y};
  asm volatile("global_store_dwordx2 %0, %1, off\n\ts_nop 4" ::"v"(p), "v"(w) : "memory");
}
__device__ __forceinline__ void str_st1(void *p, uint32_t v) {
  asm volatile("global_store_byte %0, %1, off\n\ts_nop 4" ::"v"(p), "v"(v) : "memory");
}

// LDS-DMA of 16 bytes per lane from sbase + voff (wavefront-uniform base, 32-bit lane offset) to
// LDS byte address la + 16 l. Inline assembly, so that the compiler does not make later LDS reads
// wait for it; the kernel counts its own DMAs with vm_wait.
__device__ __forceinline__ void str_dma16(uint32_t voff, const void *sbase, uint32_t la) {
  la = __builtin_amdgcn_readfirstlane(la);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(la) : "memory", "m0");
}
// The same with the non-temporal cache policy (weights read once per launch).
__device__ __forceinline__ void str_dma16_nt(uint32_t voff, const void *sbase, uint32_t la) {
  la = __builtin_amdgcn_readfirstlane(la);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase), "s"(la) : "memory", "m0");
}
// LDS-DMA of 4 bytes per lane (lane l's bytes land at la + 4 l).
__device__ __forceinline__ void str_dma4(uint32_t voff, const void *sbase, uint32_t la) {
  la = __builtin_amdgcn_readfirstlane(la);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(la) : "memory", "m0");
}
__device__ __forceinline__ uint32_t str_lds(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
}

// f(integral_constant<int, i>) for i = B .. E - 1: loop positions whose index is a constant from
// the start, so every ring slot, wait count and scale-buffer index is a constant.
template <int B, int E, typename F>
__device__ __forceinline__ void str_static_for(F &&f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    str_static_for<B + 1, E>(f);
  }
}

}  // namespace moe

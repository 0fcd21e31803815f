// Direct global -> LDS loads (gfx950 global_load_lds_dword / _dwordx4) issued
// from inline asm, and the matching explicit wait.  The kernels that use them
// keep their own count of outstanding loads on the in-order vmcnt counter:
// the compiler does not see these loads, so it neither inserts conservative
// vmcnt(0) waits before LDS reads nor accounts them -- the caller waits with
// wait_vm_barrier<N>() (N = loads issued after the ones that must be done)
// before reading what they wrote.
#pragma once

#include "ti_common.h"

namespace ti {

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// 16 bytes per lane: global g -> LDS at lds_base + 16 * lane (lds_base is
// wave-uniform; M0 carries it).
__device__ __forceinline__ void dma16(const void* g, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_base))
               : "memory");
}

// 16 bytes per lane from a wave-uniform base plus a 32-bit per-lane byte offset
// (the scalar-base form: the base lives in SGPRs, so a loop that only moves the
// base spends no vector instructions on addresses).
__device__ __forceinline__ void dma16_sv(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "s"(__builtin_amdgcn_readfirstlane(lds_base))
               : "memory");
}

// 4 bytes per lane: global g -> LDS at lds_base + 4 * lane.
__device__ __forceinline__ void dma4(const void* g, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :
               : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_base))
               : "memory");
}

// Wait until at most N of this wave's vector-memory loads are outstanding,
// then barrier the workgroup.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(N) : "memory");
}

__device__ __forceinline__ void wait_vm_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

}  // namespace ti

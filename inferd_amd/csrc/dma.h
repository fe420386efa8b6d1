// Direct global -> LDS loads and the wait + barrier that closes a pipeline stage (gfx950).
#pragma once
#include <hip/hip_runtime.h>

namespace ifd {

typedef __attribute__((address_space(3))) void lds_void_t;

// One wave-wide 16-byte-per-lane DMA (global_load_lds_dwordx4): lane l's 16 bytes land at lds + 16 l. The LDS base
// goes to M0, one value per wave: issue it under wave-uniform control flow only (under a lane-dependent branch the
// compiler may merge two such loads and keep one M0 for both).
__device__ __forceinline__ void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_void_t*)lds, 16, 0, 0);
}
// Wait until at most N DMA/vector loads of this wave are outstanding and all its LDS reads are done, then barrier.
// One asm statement with a memory clobber: the compiler may not move LDS accesses across it, and it adds no wait of
// its own (a __syncthreads() would drain every outstanding DMA).
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

}  // namespace ifd

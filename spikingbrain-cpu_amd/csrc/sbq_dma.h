// sbq_dma.h - global -> LDS copy helpers and waits shared by the tiled GEMM
// GEMM kernels (sbq_gemm.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sbq {

// LDS activation tile for s8 operands: 64 bytes per row = 4 chunks.
__device__ __forceinline__ int xq_off(int row, int chunk) { return row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4); }

// Raw buffer over [base, base + bytes): loads outside it return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// 16 bytes per lane from buffer offset voff + soff straight into LDS at
// lds + 16 * lane (lds wave-uniform).
__device__ __forceinline__ void lds_dma16_buf(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff, void* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// Cache policy of buffer accesses that other XCDs read or wrote (sc1: coherent
// at device scope without an L2 write-back or invalidate).
constexpr int kCoherent = 16;


// s_waitcnt vmcnt(n) (n < 64) leaving the other counters unconstrained.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// Workgroup barrier without the release/acquire fence of __syncthreads():
// the fence would wait for every outstanding load, including the LDS DMA of
// the stages still in flight.  Each wave waits for its own DMA of the stage it
// is about to read (wait_vmcnt) before arriving here; the asm clobbers keep
// the compiler from moving LDS accesses across the barrier.
__device__ __forceinline__ void barrier_nofence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace sbq

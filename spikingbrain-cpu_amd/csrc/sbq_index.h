// sbq_index.h - index arithmetic of the kernels that a host-side bounds check
// also compiles (plain C++: no HIP types or builtins here).  Each function maps
// a work item to the element or byte range it reads or writes; the kernels use
// these functions, and tests/bounds_check.cpp walks every work item of a
// launch through them with g++ and checks the ranges against the buffers.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define SBQ_HD __host__ __device__ __forceinline__
#else
#define SBQ_HD inline
#endif

namespace sbq {

// Activation quantizer, vector path (K % 16 == 0, Kp = ceil(K / 64) * 64):
// 16-element chunk c of x [M, K] (row stride ldx), cpr = Kp / 16 chunks per
// row.  Returns the element offset of the first of the 16 values loaded.
// Chunks in the padding columns K..Kp-1 load the row's last chunk (their
// values are never used), so no load leaves the row.
SBQ_HD int64_t act_chunk_src(int64_t c, int cpr, int K, int64_t ldx) {
  const int64_t m = c / cpr;
  const int k0 = (int)(c - m * cpr) * 16;
  return m * ldx + (k0 < K - 16 ? k0 : K - 16);
}

}  // namespace sbq

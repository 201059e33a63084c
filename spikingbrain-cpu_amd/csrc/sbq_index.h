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

// Greedy-token key of output value v at column n (fused argmax of the decode
// GEMV).  The unsigned 64-bit order of keys is torch.argmax's order of
// (value, index): NaN above every number, -0 equal to +0, and among equal
// values the smaller index.  Key 0 is below every key (no candidate).
SBQ_HD unsigned long long argmax_key(float v, int n) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  if (v != v) {
    u = 0xffffffffu;
  } else if (v == 0.0f) {
    u = 0x80000000u;  // -0 and +0 alike
  } else {
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  }
  return ((unsigned long long)u << 32) | (unsigned long long)(0xffffffffu - (uint32_t)n);
}

// Workgroups b < nblk with b % slots == slot (the fused argmax's members of
// one slot), and the number of slots that have any.
SBQ_HD unsigned argmax_slot_members(unsigned nblk, unsigned slot, unsigned slots) {
  return slot < nblk ? (nblk - slot + slots - 1) / slots : 0u;
}
SBQ_HD unsigned argmax_slots_used(unsigned nblk, unsigned slots) { return nblk < slots ? nblk : slots; }

// Column index of a key from argmax_key.
SBQ_HD int argmax_key_index(unsigned long long key) { return (int)(0xffffffffu - (uint32_t)key); }

}  // namespace sbq

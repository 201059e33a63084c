// sbq_gemv_ops.h - activation fragments and MFMA steps shared by the decode
// GEMV kernels (sbq_gemv.hip: general shapes; sbq_gemv_fast.hip: the common
// aligned case).
#pragma once
#include <type_traits>

#include "sbq_common.h"

namespace sbq {

// Arguments of the decode GEMV kernels (one struct, passed by value).
// One linear of a grouped decode launch: its operands and the first
// workgroup of its share of the grid.
struct GemvSeg {
  const void* x;
  const uint8_t* packed;
  const float* scale;
  const float* bias;
  const int32_t* colsum;  // int8-dyn: the weight column sums
  void* y;
  int64_t ldx, ldy;
  int N, Nt, wg0, pad;
};
constexpr int kGemvMaxSeg = 4;  // linears per grouped launch

struct GemvArgs {
  const void* x;
  int64_t ldx;
  int M, K, Kc;
  const uint8_t* packed;
  const float* scale;
  const float* bias;
  const int32_t* colsum;
  int N, Nt, ngroups;
  void* y;
  int yt;
  int64_t ldy;
  int32_t* acc_out;
  const float2* partials;
  int nparts;
  const float* rscale;  // per-token W8A8: s_t [M]
  const float* qpbuf;   // W8A8 on pre-quantized rows: (s_x, zp bits) from the quantize pre-pass
  int flags;            // kGemvXVec | kGemvYVec | kGemvArgmax
  // greedy token of each row (flags & kGemvArgmax; fp32 y): the argmax state
  // (per-slot keys and counts, zero before the launch and zero again after
  // it) and the int64 token per row
  uint8_t* am_state;
  int64_t* idx;
  // grouped launch (fast path, weight-only or int8-dyn with the activation
  // min/max reduced in the kernel): nseg > 1 independent linears of
  // the same M, K and dtypes; workgroup b belongs to the last segment s with
  // seg[s].wg0 <= b and takes its operands (the fields above describe none)
  int nseg;
  GemvSeg seg[kGemvMaxSeg];
};
// The fused argmax's state: kArgmaxSlots slots of 16 row keys (128 bytes) and
// a count, kArgmaxSlotBytes apart, then the count of finished slots.
constexpr int kArgmaxSlots = 64;
constexpr int kArgmaxSlotBytes = 256;
constexpr int kArgmaxStateBytes = (kArgmaxSlots + 1) * kArgmaxSlotBytes;
constexpr int kGemvXVec = 1;     // x rows 16-byte aligned: vector loads
constexpr int kGemvYVec = 2;     // y rows aligned for 4-element vector stores
constexpr int kGemvArgmax = 4;   // also pick each row's argmax (fused greedy token)
constexpr int kGemvPerToken = 8; // W8A8 per-token symmetric, x quantized in the kernel (rows, M <= 16)

// ---------------------------------------------------------------------------
// Raw activations of one lane: x[m][k0 .. k0+15], m = mt*16 + r,
// k0 = kc*64 + g*16.  Rows >= M and columns >= K read as zero.
// ---------------------------------------------------------------------------
template <int XT>
struct XRaw;

// 16 pre-quantized s8 activations: the i8 MFMA B operand as loaded
template <>
struct XRaw<XT_S8> {
  u32x4 v;
};

template <>
struct XRaw<XT_F16> {
  f16x8 a, b;
  __device__ __forceinline__ void load(const void* x, int64_t ldx, int M, int K, int m, int k0, bool xvec) {
    const _Float16* p = (const _Float16*)x + (int64_t)m * ldx + k0;
    if (m < M && xvec && k0 + 16 <= K) {
      a = *(const f16x8*)p;
      b = *(const f16x8*)(p + 8);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        a[j] = (m < M && k0 + j < K) ? p[j] : (_Float16)0.0f;
        b[j] = (m < M && k0 + 8 + j < K) ? p[8 + j] : (_Float16)0.0f;
      }
    }
  }
  __device__ __forceinline__ float get(int j) const { return j < 8 ? (float)a[j] : (float)b[j - 8]; }
  __device__ __forceinline__ void load_lds(const uint8_t* xl, int Kp, int M, int m, int k0) {
    if (m < M) {
      const _Float16* p = (const _Float16*)xl + m * Kp + k0;
      a = *(const f16x8*)p;
      b = *(const f16x8*)(p + 8);
    } else {
      a = f16x8{};
      b = f16x8{};
    }
  }
};

template <>
struct XRaw<XT_BF16> {
  bf16x8 a, b;
  __device__ __forceinline__ void load(const void* x, int64_t ldx, int M, int K, int m, int k0, bool xvec) {
    const __bf16* p = (const __bf16*)x + (int64_t)m * ldx + k0;
    if (m < M && xvec && k0 + 16 <= K) {
      a = *(const bf16x8*)p;
      b = *(const bf16x8*)(p + 8);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        a[j] = (m < M && k0 + j < K) ? p[j] : (__bf16)0.0f;
        b[j] = (m < M && k0 + 8 + j < K) ? p[8 + j] : (__bf16)0.0f;
      }
    }
  }
  __device__ __forceinline__ float get(int j) const { return j < 8 ? (float)a[j] : (float)b[j - 8]; }
  __device__ __forceinline__ void load_lds(const uint8_t* xl, int Kp, int M, int m, int k0) {
    if (m < M) {
      const __bf16* p = (const __bf16*)xl + m * Kp + k0;
      a = *(const bf16x8*)p;
      b = *(const bf16x8*)(p + 8);
    } else {
      a = bf16x8{};
      b = bf16x8{};
    }
  }
};

template <>
struct XRaw<XT_F32> {
  f32x4 v[4];
  __device__ __forceinline__ void load(const void* x, int64_t ldx, int M, int K, int m, int k0, bool xvec) {
    const float* p = (const float*)x + (int64_t)m * ldx + k0;
    if (m < M && xvec && k0 + 16 <= K) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = *(const f32x4*)(p + 4 * i);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j >> 2][j & 3] = (m < M && k0 + j < K) ? p[j] : 0.0f;
    }
  }
  __device__ __forceinline__ float get(int j) const { return v[j >> 2][j & 3]; }
  __device__ __forceinline__ void load_lds(const uint8_t* xl, int Kp, int M, int m, int k0) {
    if (m < M) {
      const float* p = (const float*)xl + m * Kp + k0;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = *(const f32x4*)(p + 4 * i);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = f32x4{};
    }
  }
};

// Element bytes of an activation type.
template <int XT>
constexpr int x_bytes() { return XT == XT_F32 ? 4 : (XT == XT_S8 ? 1 : 2); }

// Default number of 16-byte chunks of x per thread the LDS staging holds.
constexpr int kStageChunks = 4;

// Weight tile (16 offset-binary bytes of one lane) x activation fragment ->
// MFMA into acc.  fp16/bf16 activations are exact operands; fp32 activations
// run as bf16 hi + bf16 remainder (two passes, remainder first).
template <int XT>
__device__ __forceinline__ void tile_mma(u32x4 w, const XRaw<XT>& x, f32x4& acc) {
  if constexpr (XT == XT_F16) {
    f16x8 w0, w1;
    u8x16_to_f16(w, w0, w1);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(w0, x.a, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(w1, x.b, acc, 0, 0, 0);
  } else if constexpr (XT == XT_BF16) {
    bf16x8 w0, w1;
    u8x16_to_bf16(w, w0, w1);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0, x.a, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1, x.b, acc, 0, 0, 0);
  } else {
    bf16x8 w0, w1, h0, h1, l0, l1;
    u8x16_to_bf16(w, w0, w1);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      __bf16 h, l;
      split_bf16(x.get(j), h, l);
      h0[j] = h;
      l0[j] = l;
      split_bf16(x.get(8 + j), h, l);
      h1[j] = h;
      l1[j] = l;
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0, l0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1, l1, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0, h0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1, h1, acc, 0, 0, 0);
  }
}

// s8 activation fragment (xq - 128) from raw values; columns >= K and rows
// >= M become 0 (they meet zero weights or are never stored).
template <int XT>
__device__ __forceinline__ i32x4 quant_frag(const XRaw<XT>& x, int M, int K, int m, int k0, float inv, float zpf) {
  uint32_t d[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float t[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int jj = 4 * i + j;
      // outside x: xq = 128, i.e. s8 0
      t[j] = (m < M && k0 + jj < K) ? __builtin_fmaf(x.get(jj), inv, zpf) : 128.0f;
    }
    d[i] = pack_act_s8x4(t[0], t[1], t[2], t[3]);
  }
  return (i32x4){(int)d[0], (int)d[1], (int)d[2], (int)d[3]};
}


__device__ __forceinline__ u32x4 load_tile_nt(const uint8_t* p) {
  return __builtin_nontemporal_load((const u32x4*)p);
}

}  // namespace sbq

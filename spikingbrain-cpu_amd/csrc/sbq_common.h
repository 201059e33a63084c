// sbq_common.h - device helpers shared by the gfx950 quantized-linear kernels.
//
// Operand conventions (all kernels):
//   * weights live in the packed 16x64 tile layout of include/sbq.h: one 1 KiB
//     tile is one wavefront load of 16 bytes per lane, lane = g*16 + r holds
//     row r (0..15) and columns g*16..g*16+15 of the tile, stored offset-binary
//     (u = q + 128).
//   * the MFMA A operand is always the weight fragment (MFMA row = output
//     channel n) and the B operand the activation fragment (MFMA column =
//     token m), so D = W * X^T and lane l of a 16x16 accumulator holds
//     y[m = l%16][n = 4*(l/16) + v], v = 0..3: four consecutive outputs of one
//     token, which the epilogue stores as one vector.
//   * a lane's K positions inside a 64-wide tile are g*16 + 8*s + (0..7) for
//     MFMA step s = 0,1 (16x16x32) or g*16 + (0..15) (16x16x64 i8); weights and
//     activations use the same assignment, so the product is the dot product
//     whatever K slot order the instruction uses internally.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sbq {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

enum XType { XT_F32 = 0, XT_F16 = 1, XT_BF16 = 2, XT_S8 = 3 };  // XT_S8: pre-quantized activations (internal)

// ---------------------------------------------------------------------------
// int8 (offset binary) -> fp16 / bf16, exact.
// ---------------------------------------------------------------------------

// 4 offset-binary bytes -> 4 fp16 values q = u - 128.
// v_perm_b32 builds the fp16 bit patterns 0x6400 | u (= 1024 + u, exact since
// fp16 has unit spacing on [1024, 2048)); one packed subtract of 1152 leaves q.
__device__ __forceinline__ void u8x4_to_f16(uint32_t w, f16x2& lo, f16x2& hi) {
  const uint32_t a = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);
  const uint32_t b = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);
  const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  lo = __builtin_bit_cast(f16x2, a) - bias;
  hi = __builtin_bit_cast(f16x2, b) - bias;
}

// 8 offset-binary bytes u = q + 128 -> 8 fp16 subnormals u * 2^-24 (exact,
// one v_perm per pair of values).  The caller removes the offset:
// sum_k u_k x_k = 2^24 * sum_k (q_k x_k) * 2^-24 + 128 * sum_k x_k.
__device__ __forceinline__ f16x8 u8x8_to_f16_sub(uint32_t lo, uint32_t hi) {
  const u32x4 d = {__builtin_amdgcn_perm(0u, lo, 0x0c010c00u), __builtin_amdgcn_perm(0u, lo, 0x0c030c02u),
                   __builtin_amdgcn_perm(0u, hi, 0x0c010c00u), __builtin_amdgcn_perm(0u, hi, 0x0c030c02u)};
  return __builtin_bit_cast(f16x8, d);
}

// 16 offset-binary bytes (one lane slot of a tile) -> two fp16 MFMA operands:
// s0 = columns 0..7, s1 = columns 8..15 of the slot.
__device__ __forceinline__ void u8x16_to_f16(u32x4 w, f16x8& s0, f16x8& s1) {
  f16x2 p0, p1, p2, p3, p4, p5, p6, p7;
  u8x4_to_f16(w.x, p0, p1);
  u8x4_to_f16(w.y, p2, p3);
  u8x4_to_f16(w.z, p4, p5);
  u8x4_to_f16(w.w, p6, p7);
  s0 = (f16x8){p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
  s1 = (f16x8){p4.x, p4.y, p5.x, p5.y, p6.x, p6.y, p7.x, p7.y};
}

// 4 offset-binary bytes -> 4 bf16 values q (|q| <= 128 has <= 8 significant
// bits, so every conversion below is exact).  One xor turns the four bytes
// into q as signed bytes; each then converts with one sign-extending
// sub-dword convert (no separate subtract of the offset).
__device__ __forceinline__ void u8x4_to_bf16(uint32_t w, __bf16* out) {
  const uint32_t s = w ^ 0x80808080u;
  out[0] = (__bf16)(float)(int8_t)s;
  out[1] = (__bf16)(float)(int8_t)(s >> 8);
  out[2] = (__bf16)(float)(int8_t)(s >> 16);
  out[3] = (__bf16)(float)(int8_t)(s >> 24);
}

__device__ __forceinline__ void u8x16_to_bf16(u32x4 w, bf16x8& s0, bf16x8& s1) {
  __bf16 t[16];
  u8x4_to_bf16(w.x, t + 0);
  u8x4_to_bf16(w.y, t + 4);
  u8x4_to_bf16(w.z, t + 8);
  u8x4_to_bf16(w.w, t + 12);
  s0 = (bf16x8){t[0], t[1], t[2], t[3], t[4], t[5], t[6], t[7]};
  s1 = (bf16x8){t[8], t[9], t[10], t[11], t[12], t[13], t[14], t[15]};
}

// 16 offset-binary weight bytes of a packed tile -> s8 MFMA operand (q).
__device__ __forceinline__ i32x4 tile_to_s8(u32x4 w) {
  return (i32x4){(int)(w.x ^ 0x80808080u), (int)(w.y ^ 0x80808080u), (int)(w.z ^ 0x80808080u),
                 (int)(w.w ^ 0x80808080u)};
}

// ---------------------------------------------------------------------------
// Activation element access
// ---------------------------------------------------------------------------
template <int XT>
struct XElem;
template <>
struct XElem<XT_F32> {
  typedef float T;
  static __device__ __forceinline__ float to_f32(float v) { return v; }
};
template <>
struct XElem<XT_F16> {
  typedef _Float16 T;
  static __device__ __forceinline__ float to_f32(_Float16 v) { return (float)v; }
};
template <>
struct XElem<XT_BF16> {
  typedef __bf16 T;
  static __device__ __forceinline__ float to_f32(__bf16 v) { return (float)v; }
};

// 8 consecutive activations x[m][k0..k0+7] widened to fp32.  `vec` = the row
// is 16-byte aligned at k0 and all 8 columns are < K; otherwise each element is
// loaded alone and columns >= K read as zero.  Rows >= M read as zero.
template <int XT>
__device__ __forceinline__ void load8_f32(const void* x, int64_t ldx, int M, int K, int m, int k0, bool vec,
                                          float* t) {
  typedef typename XElem<XT>::T T;
  const T* p = (const T*)x + (int64_t)m * ldx + k0;
  if (m < M && vec && k0 + 8 <= K) {
    if constexpr (XT == XT_F32) {
      const f32x4 a = *(const f32x4*)p;
      const f32x4 b = *(const f32x4*)(p + 4);
      t[0] = a.x; t[1] = a.y; t[2] = a.z; t[3] = a.w;
      t[4] = b.x; t[5] = b.y; t[6] = b.z; t[7] = b.w;
    } else {
      typedef T v8 __attribute__((ext_vector_type(8)));
      const v8 a = *(const v8*)p;
#pragma unroll
      for (int j = 0; j < 8; ++j) t[j] = XElem<XT>::to_f32(a[j]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = (m < M && k0 + j < K) ? XElem<XT>::to_f32(p[j]) : 0.0f;
  }
}

// 8 consecutive activations at p (16-byte aligned, all in bounds) widened to
// fp32, with no guard.
template <int XT>
__device__ __forceinline__ void load8_f32_vec(const typename XElem<XT>::T* p, float* t) {
  typedef typename XElem<XT>::T T;
  if constexpr (XT == XT_F32) {
    const f32x4 a = *(const f32x4*)p;
    const f32x4 b = *(const f32x4*)(p + 4);
    t[0] = a.x; t[1] = a.y; t[2] = a.z; t[3] = a.w;
    t[4] = b.x; t[5] = b.y; t[6] = b.z; t[7] = b.w;
  } else {
    typedef T v8 __attribute__((ext_vector_type(8)));
    const v8 a = *(const v8*)p;
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = XElem<XT>::to_f32(a[j]);
  }
}

// fp32 -> (hi, lo) bf16 pair with hi + lo == v to 16 significant bits.
__device__ __forceinline__ void split_bf16(float v, __bf16& hi, __bf16& lo) {
  hi = (__bf16)v;
  lo = (__bf16)(v - (float)hi);
}

// Exponent e of the power-of-two row scale that puts a row's largest
// magnitude mx into [2^14, 2^15) before the row is rounded to fp16
// (exact scaling; no fp16 overflow, at most 2^28 of range lost to
// subnormals below the maximum).  Rows with no finite nonzero maximum keep
// e = 0.
__device__ __forceinline__ int row_scale_exp(float mx) {
  int e = 0;
  if (mx > 0.0f && mx <= 3.4028235e38f) {
    int ex;
    (void)frexpf(mx, &ex);  // mx in [2^(ex-1), 2^ex)
    e = min(max(15 - ex, -112), 120);
  }
  return e;
}

// ---------------------------------------------------------------------------
// Output element store
// ---------------------------------------------------------------------------
// fp32 -> 2-byte conversion of a computed output.  The empty asm hides how the
// value was produced, so the compiler cannot fuse the final fma / add with the
// conversion into one mixed-precision instruction (v_fma_mixlo_f16) that
// rounds the exact result once to 16 bits: a 2-byte output is the fp32 result
// rounded again, as converting the reference's fp32 output is.
__device__ __forceinline__ float fp32_rounded(float v) {
  asm("" : "+v"(v));
  return v;
}
__device__ __forceinline__ _Float16 out_f16(float v) { return (_Float16)fp32_rounded(v); }
__device__ __forceinline__ __bf16 out_bf16(float v) { return (__bf16)fp32_rounded(v); }

__device__ __forceinline__ void store_y(void* y, int ytype, int64_t idx, float v) {
  if (ytype == XT_F32) {
    ((float*)y)[idx] = v;
  } else if (ytype == XT_F16) {
    ((_Float16*)y)[idx] = out_f16(v);
  } else {
    ((__bf16*)y)[idx] = out_bf16(v);
  }
}

// Two 2-byte values in one dword, element 0 in the low half.
__device__ __forceinline__ uint32_t pack_h2(_Float16 a, _Float16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}
__device__ __forceinline__ uint32_t pack_b2(__bf16 a, __bf16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// Four consecutive outputs; `vec` says the 4-element group is in range and
// aligned for one vector store.
__device__ __forceinline__ void store_y4(void* y, int ytype, int64_t idx, f32x4 v, bool vec, int nvalid) {
  if (vec) {
    if (ytype == XT_F32) {
      *(f32x4*)((float*)y + idx) = v;
    } else if (ytype == XT_F16) {
      typedef _Float16 h4 __attribute__((ext_vector_type(4)));
      h4 h = {out_f16(v.x), out_f16(v.y), out_f16(v.z), out_f16(v.w)};
      *(h4*)((_Float16*)y + idx) = h;
    } else {
      typedef __bf16 b4 __attribute__((ext_vector_type(4)));
      b4 h = {out_bf16(v.x), out_bf16(v.y), out_bf16(v.z), out_bf16(v.w)};
      *(b4*)((__bf16*)y + idx) = h;
    }
  } else {
    if (nvalid > 0) store_y(y, ytype, idx + 0, v.x);
    if (nvalid > 1) store_y(y, ytype, idx + 1, v.y);
    if (nvalid > 2) store_y(y, ytype, idx + 2, v.z);
    if (nvalid > 3) store_y(y, ytype, idx + 3, v.w);
  }
}

// ---------------------------------------------------------------------------
// Wave reductions
// ---------------------------------------------------------------------------
// Minimum / maximum over the wave's 64 lanes by DPP lane moves, with no LDS
// round trip: within quads, rows of 16 (half mirror, mirror), then row 0 into
// row 1 and row 2 into row 3 (row_bcast:15), rows 0-1 into rows 2-3
// (row_bcast:31); lane 63 ends with the result, which every lane then reads.
// NaN inputs are ignored (fminf / fmaxf).  Called by whole waves.
template <int CTRL, int ROWS, bool MAX>
__device__ __forceinline__ float dpp_minmax_step(float v) {
  const float t = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROWS, 0xf,
                                                             false));
  return MAX ? fmaxf(v, t) : fminf(v, t);
}
template <bool MAX>
__device__ __forceinline__ float wave_minmax(float v) {
  v = dpp_minmax_step<0xb1, 0xf, MAX>(v);   // quad_perm [1, 0, 3, 2]
  v = dpp_minmax_step<0x4e, 0xf, MAX>(v);   // quad_perm [2, 3, 0, 1]
  v = dpp_minmax_step<0x141, 0xf, MAX>(v);  // row_half_mirror
  v = dpp_minmax_step<0x140, 0xf, MAX>(v);  // row_mirror
  v = dpp_minmax_step<0x142, 0xa, MAX>(v);  // row_bcast:15
  v = dpp_minmax_step<0x143, 0xc, MAX>(v);  // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_max(float v) { return wave_minmax<true>(v); }
__device__ __forceinline__ float wave_min(float v) { return wave_minmax<false>(v); }
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ---------------------------------------------------------------------------
// fbgemm / PyTorch ChooseQuantizationParams for uint8 [0, 255] activations,
// evaluated on the device in the same double/float steps as the CPU library.
// ---------------------------------------------------------------------------
struct ActQParams {
  float scale;
  float inv;   // 1.0f / scale (IEEE fp32 division)
  float zpf;   // zero point as float (exact)
  int zp;
};

__device__ inline ActQParams choose_act_qparams(float xmin, float xmax) {
  const int qmin = 0, qmax = 255;
  const float kSmall = 6.1e-5f;
  float lo = xmin < 0.0f ? xmin : 0.0f;
  float hi = xmax > 0.0f ? xmax : 0.0f;
  double scale = ((double)hi - (double)lo) / (double)(qmax - qmin);
  float fs = (float)scale;
  if (fs == 0.0f || __builtin_isinf(1.0f / fs)) scale = 0.1;
  if (scale < (double)kSmall) {
    float org = (float)scale;
    scale = (double)kSmall;
    if (lo == 0.0f) {
      hi = kSmall * (float)(qmax - qmin);
    } else if (hi == 0.0f) {
      lo = -kSmall * (float)(qmax - qmin);
    } else {
      float amp = kSmall / org;
      lo = lo * amp;
      hi = hi * amp;
    }
  }
  double zmin = (double)qmin - (double)lo / scale;
  double zmax = (double)qmax - (double)hi / scale;
  double emin = __builtin_fabs((double)qmin) - __builtin_fabs((double)lo / scale);
  double emax = __builtin_fabs((double)qmax) - __builtin_fabs((double)hi / scale);
  double z0 = emin < emax ? zmin : zmax;
  int zp;
  if (z0 < qmin) zp = qmin;
  else if (z0 > qmax) zp = qmax;
  else zp = (int)__builtin_rint(z0);
  ActQParams p;
  p.scale = (float)scale;
  p.inv = 1.0f / p.scale;
  p.zpf = (float)zp;
  p.zp = zp;
  return p;
}

// fbgemm's activation quantizer xq = clamp(rint(fma(x, 1/s_x, zp)), 0, 255),
// kept as s8 xq - 128: four pre-rounding values t = fma(x, inv, zp) -> four
// packed bytes.  v_cvt_pk_u8_f32 computes clamp(rint(t), 0, 255) (ties to
// even, NaN -> 0; checked on MI355X) and packs the byte; ^ 0x80 maps u8 to
// s8 - 128 for four values at once.
__device__ __forceinline__ uint32_t pack_act_s8x4(float t0, float t1, float t2, float t3) {
  uint32_t w = __builtin_amdgcn_cvt_pk_u8_f32(t0, 0, 0u);
  w = __builtin_amdgcn_cvt_pk_u8_f32(t1, 1, w);
  w = __builtin_amdgcn_cvt_pk_u8_f32(t2, 2, w);
  w = __builtin_amdgcn_cvt_pk_u8_f32(t3, 3, w);
  return w ^ 0x80808080u;
}

// Number of min/max partials the activation pre-pass writes (upper bound).
constexpr int kMinMaxPartials = 256;

// Reduce the min/max partials at the start of a W8A8 kernel (every block does
// it redundantly; partials are few).  Must be called by all threads of the
// block; `red` is >= 2 * (blockDim.x / 64) floats of LDS.
__device__ inline ActQParams block_qparams_from_partials(const float2* partials, int nparts, float* red) {
  float mn = 0.0f, mx = 0.0f;  // lo <= 0 <= hi always holds after clamping
  for (int i = threadIdx.x; i < nparts; i += blockDim.x) {
    float2 p = partials[i];
    mn = fminf(mn, p.x);
    mx = fmaxf(mx, p.y);
  }
  mn = wave_min(mn);
  mx = wave_max(mx);
  const int wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[2 * wid] = mn;
    red[2 * wid + 1] = mx;
  }
  __syncthreads();
  mn = red[0];
  mx = red[1];
  for (int w = 1; w < nw; ++w) {
    mn = fminf(mn, red[2 * w]);
    mx = fmaxf(mx, red[2 * w + 1]);
  }
  __syncthreads();
  return choose_act_qparams(mn, mx);
}

}  // namespace sbq

// sbq_quant.hip - weight quantization, packing and activation statistics.
//
//   quantize_per_channel  (spikingbrain_cpu/quant.py:25-29)
//   repack / unpack / colsum (the device-side form of the buffers built by
//                            quant.py:33-39 and the prepack of quant.py:57-61)
//   activation min/max partials (first step of fbgemm's dynamic quantization,
//                                reached from quant.py:65)
#include "sbq_common.h"
#include "sbq_launch.h"

namespace sbq {

// One wavefront per weight row: exact max|w| reduction, then IEEE fp32
// divisions and round-half-even, matching torch's CPU expression.
template <int WT>
__global__ __launch_bounds__(256) void quantize_per_channel_kernel(const void* __restrict__ wv, int64_t N,
                                                                   int64_t K, int64_t ldw,
                                                                   int8_t* __restrict__ q, int64_t ldq,
                                                                   float* __restrict__ scale) {
  typedef typename XElem<WT>::T T;
  const T* w = (const T*)wv;
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const T* row = w + n * ldw;
  float amax = 0.0f;
  for (int64_t k = lane; k < K; k += 64) amax = fmaxf(amax, __builtin_fabsf(XElem<WT>::to_f32(row[k])));
  amax = wave_max(amax);
  const float s = fmaxf(amax, 1e-8f) / 127.0f;
  if (lane == 0) scale[n] = s;
  int8_t* qrow = q + n * ldq;
  for (int64_t k = lane; k < K; k += 64) {
    float t = __builtin_rintf(XElem<WT>::to_f32(row[k]) / s);
    t = fminf(fmaxf(t, -127.0f), 127.0f);
    qrow[k] = (int8_t)(int)t;
  }
}

// One thread per 16-byte lane slot of the packed layout.
__global__ __launch_bounds__(256) void repack_kernel(const int8_t* __restrict__ q, int64_t N, int64_t K,
                                                     int64_t ldq, int64_t Kc, int64_t nslots,
                                                     uint8_t* __restrict__ packed) {
  const int64_t slot = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (slot >= nslots) return;
  const int lane = (int)(slot & 63);
  const int64_t tile = slot >> 6;
  const int64_t nt = tile / Kc, kc = tile % Kc;
  const int64_t n = nt * 16 + (lane & 15);
  const int64_t k0 = kc * 64 + (lane >> 4) * 16;
  uint32_t d[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t k = k0 + i * 4 + j;
      const uint32_t b = (n < N && k < K) ? (uint32_t)(uint8_t)q[n * ldq + k] : 0u;
      word |= ((b ^ 0x80u) & 0xffu) << (8 * j);
    }
    d[i] = word;
  }
  *(u32x4*)(packed + slot * 16) = (u32x4){d[0], d[1], d[2], d[3]};
}

__global__ __launch_bounds__(256) void unpack_kernel(const uint8_t* __restrict__ packed, int64_t N, int64_t K,
                                                     int64_t Kc, int8_t* __restrict__ q, int64_t ldq) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= N * K) return;
  const int64_t n = idx / K, k = idx % K;
  const int64_t nt = n >> 4, r = n & 15, kc = k >> 6, g = (k & 63) >> 4, j = k & 15;
  const uint8_t u = packed[((nt * Kc + kc) * 64 + g * 16 + r) * 16 + j];
  q[n * ldq + k] = (int8_t)(u ^ 0x80u);
}

// colsum[n] = sum_k q[n,k]  (exact int32: |sum| <= 127 * K).
__global__ __launch_bounds__(256) void colsum_kernel(const int8_t* __restrict__ q, int64_t N, int64_t K,
                                                     int64_t ldq, int32_t* __restrict__ colsum) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  int s = 0;
  for (int64_t k = lane; k < K; k += 64) s += (int)q[n * ldq + k];
  s = wave_sum_i(s);
  if (lane == 0) colsum[n] = s;
}

// Zero the split-K tile counters of the GEMM that follows a pre-pass (the
// pre-pass runs first on the same stream, so the GEMM sees them zeroed).
__device__ __forceinline__ void zero_counters(uint32_t* c, int n) {
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < n; i += blockDim.x) c[i] = 0u;
}

// The block's (min, max) into partials[blockIdx.x]: wave reductions, then
// thread 0 over the waves.
__device__ __forceinline__ void store_block_minmax(float mn, float mx, float2* partials) {
  __shared__ float red[32];
  mn = wave_min(mn);
  mx = wave_max(mx);
  const int wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[2 * wid] = mn;
    red[2 * wid + 1] = mx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < nw; ++w) {
      mn = fminf(mn, red[2 * w]);
      mx = fmaxf(mx, red[2 * w + 1]);
    }
    partials[blockIdx.x] = make_float2(mn, mx);
  }
}

// Dense x (ldx == K, 16-byte aligned, K % 8 == 0): the M*K values are one flat
// array of 8-value chunks (16 bytes of fp16 / bf16, 32 of fp32).  Thread t of
// the grid folds chunks t, t + T, t + 2T, ... (T threads), U loads in flight
// per round with no branch: indexes past the end are clamped to the last
// chunk, whose values are already in the range (min and max are idempotent).
// No division, no per-element guard.
template <int XT, int U>
__global__ __launch_bounds__(1024) void minmax_dense_kernel(const void* __restrict__ xv, int64_t nch,
                                                            float2* __restrict__ partials,
                                                            uint32_t* __restrict__ zero, int nzero) {
  typedef typename XElem<XT>::T T;
  typedef T v8 __attribute__((ext_vector_type(8)));
  zero_counters(zero, nzero);
  const int64_t T_ = (int64_t)gridDim.x * blockDim.x;
  float mn = 0.0f, mx = 0.0f;  // fbgemm's range always holds 0
  for (int64_t c0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c0 < nch; c0 += U * T_) {
    float t[U][8];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int64_t c = min(c0 + i * T_, nch - 1);
      if constexpr (XT == XT_F32) {
        const f32x4 a0 = *(const f32x4*)((const float*)xv + c * 8), a1 = *(const f32x4*)((const float*)xv + c * 8 + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          t[i][j] = a0[j];
          t[i][4 + j] = a1[j];
        }
      } else {
        const v8 a = *(const v8*)((const T*)xv + c * 8);
#pragma unroll
        for (int j = 0; j < 8; ++j) t[i][j] = XElem<XT>::to_f32(a[j]);
      }
    }
#pragma unroll
    for (int i = 0; i < U; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        mn = fminf(mn, t[i][j]);
        mx = fmaxf(mx, t[i][j]);
      }
  }
  store_block_minmax(mn, mx, partials);
}

// Per-block (min, max) of x [M, K] with any row stride: thread t of the grid
// covers the 8-value chunks t, t + T, ... (T threads; chunks row by row).
template <int XT>
__global__ __launch_bounds__(1024) void minmax_partial_kernel(const void* __restrict__ xv, int M, int K, int64_t ldx,
                                                              float2* __restrict__ partials, int vec,
                                                              uint32_t* __restrict__ zero, int nzero) {
  zero_counters(zero, nzero);
  const int cpr = (K + 7) / 8;
  const int64_t nch = (int64_t)M * cpr;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  float mn = 0.0f, mx = 0.0f;  // lo <= 0 <= hi after clamping anyway
  auto fold = [&](const float* t, int k0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = k0 + j < K ? t[j] : 0.0f;
      mn = fminf(mn, v);
      mx = fmaxf(mx, v);
    }
  };
  int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; c + 3 * stride < nch; c += 4 * stride) {  // four chunks in flight
    float t[4][8];
    int k0[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t ci = c + i * stride;
      const int m = (int)(ci / cpr);
      k0[i] = (int)(ci - (int64_t)m * cpr) * 8;
      load8_f32<XT>(xv, ldx, M, K, m, k0[i], vec, t[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) fold(t[i], k0[i]);
  }
  for (; c < nch; c += stride) {
    const int m = (int)(c / cpr), k0 = (int)(c - (int64_t)m * cpr) * 8;
    float t[8];
    load8_f32<XT>(xv, ldx, M, K, m, k0, vec, t);
    fold(t, k0);
  }
  store_block_minmax(mn, mx, partials);
}

__global__ __launch_bounds__(256) void qparams_kernel(const float2* __restrict__ partials, int nparts,
                                                      float* __restrict__ scale_out, int32_t* __restrict__ zp_out) {
  __shared__ float red[8];
  ActQParams p = block_qparams_from_partials(partials, nparts, red);
  if (threadIdx.x == 0) {
    *scale_out = p.scale;
    *zp_out = p.zp;
  }
}

// ---------------------------------------------------------------------------
// Row argmax of fp32 logits (greedy sampling, engine.py:30-31
// `int(logits.argmax())` over the lm_head output): the first index of the
// largest value, NaN above every number, as torch.argmax.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool arg_better(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn != bn) return vn;
  if (vn) return i < bi;
  return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ void arg_take(float v, int i, float& bv, int& bi) {
  if (arg_better(v, i, bv, bi)) {
    bv = v;
    bi = i;
  }
}

// Per-row sums of fp16 activations in fp32 (the offset the prefill GEMM's
// subnormal weight encoding adds: sum_k (q + 128) x_k = sum_k q x_k + 128 * rowsum).
// One wave per row, 16-byte loads (four in flight per lane), two accumulators;
// rows are 16-byte aligned and K % 8 == 0 on this path.
__device__ __forceinline__ void rowsum_acc(u32x4 v, float& s0, float& s1) {
  const uint32_t w0 = v.x, w1 = v.y, w2 = v.z, w3 = v.w;
  const f16x2 one = {1.0f16, 1.0f16};
  s0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w0), one, s0, false);
  s1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w1), one, s1, false);
  s0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w2), one, s0, false);
  s1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w3), one, s1, false);
}

__global__ __launch_bounds__(256) void rowsum_f16_kernel(const _Float16* __restrict__ x, int64_t ldx, int M, int K,
                                                         float* __restrict__ out, uint32_t* __restrict__ zero,
                                                         int nzero) {
  zero_counters(zero, nzero);
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= M) return;
  const _Float16* p = x + (int64_t)row * ldx;
  float s0 = 0.0f, s1 = 0.0f;
  int k = lane * 8;
  // eight loads in flight (a whole K = 4096 row in one round), then four, then
  // one; the chunks are summed in the same order whichever loop takes them
  for (; k + 7 * 512 < K; k += 8 * 512) {
    u32x4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = *(const u32x4*)(p + k + j * 512);
#pragma unroll
    for (int j = 0; j < 8; ++j) rowsum_acc(v[j], s0, s1);
  }
  for (; k + 3 * 512 < K; k += 4 * 512) {
    u32x4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = *(const u32x4*)(p + k + j * 512);
#pragma unroll
    for (int j = 0; j < 4; ++j) rowsum_acc(v[j], s0, s1);
  }
  for (; k < K; k += 512) rowsum_acc(*(const u32x4*)(p + k), s0, s1);
  float s = s0 + s1;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if (lane == 0) out[row] = s;
}

// fbgemm's per-tensor activation quantization on its own (the step inside
// quantized::linear_dynamic, quant.py:65, that the int8-dyn GEMMs fuse into
// their pre-pass): the (s_x, zp) of the min/max partials, then
// xq[m,k] = clamp(rint(fma(x[m,k], 1/s_x, zp)), 0, 255) as uint8 [M][ldq],
// the arithmetic of the GEMM path's quantize pass (without its s8 shift).
// One thread per 8 consecutive values of a row; loads clamped to the row,
// stores guarded.
template <int XT>
__global__ __launch_bounds__(256) void act_quant_u8_kernel(const void* __restrict__ x, int64_t ldx, int M, int K,
                                                           bool vec, const float2* __restrict__ partials,
                                                           int nparts, uint8_t* __restrict__ xq, int64_t ldq,
                                                           bool qvec) {
  const int cpr = (K + 7) / 8;
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t cl = min(c, (int64_t)M * cpr - 1);
  const int m = (int)(cl / cpr), k0 = (int)(cl - (int64_t)m * cpr) * 8;
  float t[8];
  load8_f32<XT>(x, ldx, M, K, m, k0, vec, t);
  __shared__ float red[8];
  const ActQParams qp = block_qparams_from_partials(partials, nparts, red);
  if (c >= (int64_t)M * cpr) return;
  uint32_t d[2];
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    uint32_t v = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_fmaf(t[4 * w], qp.inv, qp.zpf), 0, 0u);
    v = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_fmaf(t[4 * w + 1], qp.inv, qp.zpf), 1, v);
    v = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_fmaf(t[4 * w + 2], qp.inv, qp.zpf), 2, v);
    d[w] = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_fmaf(t[4 * w + 3], qp.inv, qp.zpf), 3, v);
  }
  uint8_t* dst = xq + (int64_t)m * ldq + k0;
  if (qvec && k0 + 8 <= K) {
    *(u32x2*)dst = (u32x2){d[0], d[1]};
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (k0 + j < K) dst[j] = (uint8_t)(d[j >> 2] >> (8 * (j & 3)));
  }
}

// Per-token symmetric activation quantization (the opt-in int8-dyn
// granularity): each activation row is quantized exactly as
// quantize_per_channel (spikingbrain_cpu/quant.py:25-29) quantizes a weight
// row: s = max(max_k |x|, 1e-8) / 127 (IEEE division), xq = clamp(rne(x / s),
// -127, 127).  xq rows have Kp bytes; columns K..Kp-1 are written as 0.
template <int XT>
__global__ __launch_bounds__(256) void quantize_rows_sym_kernel(const void* __restrict__ xv, int64_t ldx, int M, int K,
                                                                int Kp, int vec, int8_t* __restrict__ xq,
                                                                float* __restrict__ s_out) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= M) return;
  float amax = 0.0f;
  for (int k = lane * 8; k < K; k += 512) {
    float t[8];
    load8_f32<XT>(xv, ldx, M, K, row, k, vec, t);  // columns >= K read as 0
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, __builtin_fabsf(t[j]));
  }
  amax = wave_max(amax);
  const float sc = fmaxf(amax, 1e-8f) / 127.0f;
  if (lane == 0) s_out[row] = sc;
  int8_t* qrow = xq + (int64_t)row * Kp;
  for (int k = lane * 8; k < Kp; k += 512) {
    float t[8];
    load8_f32<XT>(xv, ldx, M, K, row, k, vec, t);
    uint32_t d[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float v = __builtin_rintf(t[j] / sc);
      v = fminf(fmaxf(v, -127.0f), 127.0f);
      d[j >> 2] |= ((uint32_t)(int)v & 0xffu) << (8 * (j & 3));
    }
    *(u32x2*)(qrow + k) = (u32x2){d[0], d[1]};  // Kp % 64 == 0 and Kp-byte rows: 8-byte aligned
  }
}

// fp32 / bf16 activations -> one power-of-two scaled fp16 plane for the fp16
// prefill GEMM.  Row m is scaled by 2^e (max|x| * 2^e in [2^14, 2^15), an
// exact scaling) and rounded once: plane row m = rn16(x * 2^e).  bf16 values
// (8 significant bits) are exact down to 2^28 below the row maximum; fp32
// values keep 11 bits (relative rounding error <= 2^-11 per value, about 3e-4
// relative L2 on the outputs, inside the 1e-3 weight-only tolerance).
// rowsum[m] = the fp32 sum of the plane's fp16 values; rscale[m] = 2^-e.  One
// wave per row; rows are 16-byte aligned and K % 64 == 0 on this path.  Rows
// of at most 512 * C values are read once, every 8-value chunk of a lane in
// flight together and held in registers for the conversion; longer rows are
// read twice (maximum, then conversion), four chunks in flight.
template <int XT, int C>
__global__ __launch_bounds__(256) void stage_act_kernel(const void* __restrict__ xv, int64_t ldx, int M, int K,
                                                        _Float16* __restrict__ xs, float* __restrict__ rowsum,
                                                        float* __restrict__ rscale, uint32_t* __restrict__ zero,
                                                        int nzero) {
  zero_counters(zero, nzero);
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= M) return;
  typedef typename XElem<XT>::T T;
  const T* xr = (const T*)xv + (int64_t)row * ldx;
  _Float16* out = xs + (int64_t)row * K;
  float mx = 0.0f, s = 0.0f;
  auto convert = [&](const float* t, float sc, int k) {
    f16x8 h;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      h[j] = (_Float16)(t[j] * sc);
      s += (float)h[j];
    }
    *(f16x8*)(out + k) = h;
  };
  int e;
  if (K <= 512 * C) {
    float t[C][8];
#pragma unroll
    for (int c = 0; c < C; ++c)  // clamped: chunks past the row repeat its last chunk, never converted
      load8_f32_vec<XT>(xr + min(lane * 8 + c * 512, K - 8), t[c]);
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(t[c][j]));
    e = row_scale_exp(wave_max(mx));
    const float sc = ldexpf(1.0f, e);
#pragma unroll
    for (int c = 0; c < C; ++c)
      if (lane * 8 + c * 512 < K) convert(t[c], sc, lane * 8 + c * 512);
  } else {
    for (int k0 = lane * 8; k0 < K; k0 += 4 * 512) {
      float t[4][8];
#pragma unroll
      for (int c = 0; c < 4; ++c) load8_f32_vec<XT>(xr + min(k0 + c * 512, K - 8), t[c]);
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(t[c][j]));
    }
    e = row_scale_exp(wave_max(mx));
    const float sc = ldexpf(1.0f, e);
    for (int k0 = lane * 8; k0 < K; k0 += 4 * 512) {
      float t[4][8];
#pragma unroll
      for (int c = 0; c < 4; ++c) load8_f32_vec<XT>(xr + min(k0 + c * 512, K - 8), t[c]);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (k0 + c * 512 < K) convert(t[c], sc, k0 + c * 512);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if (lane == 0) {
    rowsum[row] = s;
    rscale[row] = ldexpf(1.0f, -e);
  }
}

// One workgroup per row; each thread keeps four independent running bests
// and has sixteen vector loads in flight at a time (a 151936-wide row is
// three rounds of loads).
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const float* __restrict__ y, int N, int64_t ldy,
                                                           int64_t* __restrict__ out, int vec) {
  const float* row = y + (int64_t)blockIdx.x * ldy;
  float bv[4];
  int bi[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    bv[u] = -__builtin_inff();
    bi[u] = 0x7fffffff;
  }
  const int T = blockDim.x, t = threadIdx.x;
  int i0 = 0;
  if (vec) {
    const int n4 = N / 4;
    int c = t;
    for (; c + 15 * T < n4; c += 16 * T) {
      f32x4 v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = *(const f32x4*)(row + 4 * (c + u * T));
#pragma unroll
      for (int u = 0; u < 16; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j) arg_take(v[u][j], 4 * (c + u * T) + j, bv[u & 3], bi[u & 3]);
    }
    for (; c + 3 * T < n4; c += 4 * T) {
      f32x4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = *(const f32x4*)(row + 4 * (c + u * T));
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j) arg_take(v[u][j], 4 * (c + u * T) + j, bv[u], bi[u]);
    }
    for (; c < n4; c += T) {
      const f32x4 v = *(const f32x4*)(row + 4 * c);
#pragma unroll
      for (int j = 0; j < 4; ++j) arg_take(v[j], 4 * c + j, bv[0], bi[0]);
    }
    i0 = n4 * 4;
  }
  for (int i = i0 + t; i < N; i += T) arg_take(row[i], i, bv[0], bi[0]);
#pragma unroll
  for (int u = 1; u < 4; ++u) arg_take(bv[u], bi[u], bv[0], bi[0]);
  float v = bv[0];
  int i = bi[0];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) arg_take(__shfl_xor(v, o, 64), __shfl_xor(i, o, 64), v, i);
  __shared__ float sv[16];
  __shared__ int si[16];
  if ((t & 63) == 0) {
    sv[t >> 6] = v;
    si[t >> 6] = i;
  }
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < (T >> 6); ++w) arg_take(sv[w], si[w], v, i);
    out[blockIdx.x] = i;
  }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
int launch_quantize_per_channel(const void* w, int wt, int64_t N, int64_t K, int64_t ldw, int8_t* q,
                                int64_t ldq, float* scale, hipStream_t st) {
  dim3 grid((unsigned)((N + 3) / 4)), block(256);
  switch (wt) {
    case XT_F32: hipLaunchKernelGGL(quantize_per_channel_kernel<XT_F32>, grid, block, 0, st, w, N, K, ldw, q, ldq, scale); break;
    case XT_F16: hipLaunchKernelGGL(quantize_per_channel_kernel<XT_F16>, grid, block, 0, st, w, N, K, ldw, q, ldq, scale); break;
    case XT_BF16: hipLaunchKernelGGL(quantize_per_channel_kernel<XT_BF16>, grid, block, 0, st, w, N, K, ldw, q, ldq, scale); break;
    default: return -2;
  }
  return check_launch();
}

int launch_repack(const int8_t* q, int64_t N, int64_t K, int64_t ldq, uint8_t* packed, int32_t* colsum,
                  hipStream_t st) {
  const int64_t Nt = (N + 15) / 16, Kc = (K + 63) / 64;
  const int64_t nslots = Nt * Kc * 64;
  hipLaunchKernelGGL(repack_kernel, dim3((unsigned)((nslots + 255) / 256)), dim3(256), 0, st, q, N, K, ldq, Kc,
                     nslots, packed);
  int rc = check_launch();
  if (rc || !colsum) return rc;
  hipLaunchKernelGGL(colsum_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st, q, N, K, ldq, colsum);
  return check_launch();
}

int launch_unpack(const uint8_t* packed, int64_t N, int64_t K, int8_t* q, int64_t ldq, hipStream_t st) {
  const int64_t Kc = (K + 63) / 64;
  const int64_t total = N * K;
  hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, packed, N, K, Kc, q,
                     ldq);
  return check_launch();
}

int minmax_nparts(int64_t M, int64_t K) {
  const int64_t total = M * K;
  int64_t p = (total + 2047) / 2048;  // >= 8 elements per thread at the smallest block
  if (p < 1) p = 1;
  if (p > kMinMaxPartials) p = kMinMaxPartials;
  return (int)p;
}

int launch_minmax_partials(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, float2* partials,
                           int nparts, hipStream_t st, uint32_t* zero, int nzero) {
  const int esz = xt == XT_F32 ? 4 : 2;
  const int vec = ((uintptr_t)x % 16 == 0) && ((ldx * esz) % 16 == 0);
  // smaller workgroups for small x (measured at K = 4096: M = 128 3.4 -> 2.8 us,
  // M = 512 3.6 -> 3.4 us; from M = 1024 the 1024-thread workgroups are fastest)
  const int64_t total = M * K;
  const int threads = total <= ((int64_t)1 << 19) ? 256 : (total <= ((int64_t)1 << 21) ? 512 : 1024);
  dim3 grid((unsigned)nparts), block(threads);
  if (vec && ldx == K && K % 8 == 0) {  // one flat array of 8-value chunks
    const int64_t nch = total / 8;
#define SBQ_MINMAX_DENSE(XT_)                                                                                    \
  hipLaunchKernelGGL((minmax_dense_kernel<XT_, 4>), grid, block, 0, st, x, nch, partials, zero, nzero);
    switch (xt) {
      case XT_F32: SBQ_MINMAX_DENSE(XT_F32) break;
      case XT_F16: SBQ_MINMAX_DENSE(XT_F16) break;
      case XT_BF16: SBQ_MINMAX_DENSE(XT_BF16) break;
      default: return -2;
    }
#undef SBQ_MINMAX_DENSE
    return check_launch();
  }
  switch (xt) {
    case XT_F32: hipLaunchKernelGGL(minmax_partial_kernel<XT_F32>, grid, block, 0, st, x, (int)M, (int)K, ldx, partials, vec, zero, nzero); break;
    case XT_F16: hipLaunchKernelGGL(minmax_partial_kernel<XT_F16>, grid, block, 0, st, x, (int)M, (int)K, ldx, partials, vec, zero, nzero); break;
    case XT_BF16: hipLaunchKernelGGL(minmax_partial_kernel<XT_BF16>, grid, block, 0, st, x, (int)M, (int)K, ldx, partials, vec, zero, nzero); break;
    default: return -2;
  }
  return check_launch();
}

int launch_qparams(const float2* partials, int nparts, float* scale_out, int32_t* zp_out, hipStream_t st) {
  hipLaunchKernelGGL(qparams_kernel, dim3(1), dim3(256), 0, st, partials, nparts, scale_out, zp_out);
  return check_launch();
}

int launch_rowsum_f16(const void* x, int64_t ldx, int64_t M, int64_t K, float* out, hipStream_t st, uint32_t* zero,
                      int nzero) {
  hipLaunchKernelGGL(rowsum_f16_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, st, (const _Float16*)x, ldx, (int)M,
                     (int)K, out, zero, nzero);
  return check_launch();
}

int launch_stage_act(const void* x, int xt, int64_t ldx, int64_t M, int64_t K, _Float16* xs, float* rowsum,
                     float* rscale, hipStream_t st, uint32_t* zero, int nzero) {
  const dim3 grid((unsigned)((M + 3) / 4)), block(256);
  if (xt == XT_F32)
    hipLaunchKernelGGL((stage_act_kernel<XT_F32, 8>), grid, block, 0, st, x, ldx, (int)M, (int)K, xs, rowsum, rscale,
                       zero, nzero);
  else if (xt == XT_BF16)
    hipLaunchKernelGGL((stage_act_kernel<XT_BF16, 8>), grid, block, 0, st, x, ldx, (int)M, (int)K, xs, rowsum, rscale,
                       zero, nzero);
  else
    return -2;
  return check_launch();
}

int launch_act_quant_u8(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec, const float2* partials,
                        int nparts, uint8_t* xq, int64_t ldq, hipStream_t st) {
  const int64_t chunks = M * ((K + 7) / 8);
  const dim3 grid((unsigned)((chunks + 255) / 256)), block(256);
  const bool qvec = (uintptr_t)xq % 8 == 0 && ldq % 8 == 0;
  switch (xt) {
    case XT_F32: hipLaunchKernelGGL(act_quant_u8_kernel<XT_F32>, grid, block, 0, st, x, ldx, (int)M, (int)K, xvec, partials, nparts, xq, ldq, qvec); break;
    case XT_F16: hipLaunchKernelGGL(act_quant_u8_kernel<XT_F16>, grid, block, 0, st, x, ldx, (int)M, (int)K, xvec, partials, nparts, xq, ldq, qvec); break;
    case XT_BF16: hipLaunchKernelGGL(act_quant_u8_kernel<XT_BF16>, grid, block, 0, st, x, ldx, (int)M, (int)K, xvec, partials, nparts, xq, ldq, qvec); break;
    default: return -2;
  }
  return check_launch();
}

int launch_quantize_rows_sym(const void* x, int xt, int64_t ldx, bool xvec, int64_t M, int64_t K, int64_t Kp,
                             int8_t* xq, float* s_out, hipStream_t st) {
  const dim3 grid((unsigned)((M + 3) / 4)), block(256);
  const int vec = xvec ? 1 : 0;
  switch (xt) {
    case XT_F32: hipLaunchKernelGGL(quantize_rows_sym_kernel<XT_F32>, grid, block, 0, st, x, ldx, (int)M, (int)K, (int)Kp, vec, xq, s_out); break;
    case XT_F16: hipLaunchKernelGGL(quantize_rows_sym_kernel<XT_F16>, grid, block, 0, st, x, ldx, (int)M, (int)K, (int)Kp, vec, xq, s_out); break;
    case XT_BF16: hipLaunchKernelGGL(quantize_rows_sym_kernel<XT_BF16>, grid, block, 0, st, x, ldx, (int)M, (int)K, (int)Kp, vec, xq, s_out); break;
    default: return -2;
  }
  return check_launch();
}

int launch_argmax_rows(const float* y, int64_t M, int64_t N, int64_t ldy, int64_t* out, hipStream_t st) {
  const int vec = ((uintptr_t)y % 16 == 0) && (ldy % 4 == 0);
  hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)M), dim3(1024), 0, st, y, (int)N, ldy, out, vec);
  return check_launch();
}

}  // namespace sbq

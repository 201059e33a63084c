// sbq_gemv.hip - decode (small-M) quantized linear, HBM-bandwidth bound.
//
// Replaces the per-token projections of spikingbrain_cpu/quant.py:41-53
// (Int8Linear.forward, weight-only) and quant.py:63-66 (DynamicInt8Linear,
// W8A8) at the decode shapes the engine issues (engine.py:106: M = 1).
//
// Work decomposition: a workgroup owns G consecutive 16-row weight tiles and
// splits K over its waves; each wave streams its contiguous run of 1 KiB
// packed tiles (one 16-byte non-temporal load per lane per tile), converts
// them in registers and feeds MFMA 16x16 instructions with the activation
// fragment as the second operand.  The per-wave partial tiles are summed in
// LDS in a fixed wave order (deterministic), then scale/bias are applied and
// four consecutive outputs per lane are stored as one vector.
#include "sbq_common.h"
#include "sbq_launch.h"

namespace sbq {

// ---------------------------------------------------------------------------
// Activation fragments: lane (r, g) of M-tile mt holds x[mt*16 + r][k0 .. k0+15]
// with k0 = kc*64 + g*16.  Rows >= M and columns >= K read as zero.
// ---------------------------------------------------------------------------
template <int XT>
struct XFrag;

template <>
struct XFrag<XT_F16> {
  static constexpr int NS = 1;
  typedef f16x8 V;
  V v[2][1];
  __device__ __forceinline__ void load(const void* x, int64_t ldx, int M, int K, int m, int k0, bool xvec) {
    const _Float16* p = (const _Float16*)x + (int64_t)m * ldx + k0;
    if (m < M && xvec && k0 + 16 <= K) {
      v[0][0] = *(const f16x8*)p;
      v[1][0] = *(const f16x8*)(p + 8);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[0][0][j] = (m < M && k0 + j < K) ? p[j] : (_Float16)0.0f;
        v[1][0][j] = (m < M && k0 + 8 + j < K) ? p[8 + j] : (_Float16)0.0f;
      }
    }
  }
};

template <>
struct XFrag<XT_BF16> {
  static constexpr int NS = 1;
  typedef bf16x8 V;
  V v[2][1];
  __device__ __forceinline__ void load(const void* x, int64_t ldx, int M, int K, int m, int k0, bool xvec) {
    const __bf16* p = (const __bf16*)x + (int64_t)m * ldx + k0;
    if (m < M && xvec && k0 + 16 <= K) {
      v[0][0] = *(const bf16x8*)p;
      v[1][0] = *(const bf16x8*)(p + 8);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[0][0][j] = (m < M && k0 + j < K) ? p[j] : (__bf16)0.0f;
        v[1][0][j] = (m < M && k0 + 8 + j < K) ? p[8 + j] : (__bf16)0.0f;
      }
    }
  }
};

// fp32 activations: each value is split into bf16 hi + bf16 remainder, two
// MFMA passes per step.
template <>
struct XFrag<XT_F32> {
  static constexpr int NS = 2;
  typedef bf16x8 V;
  V v[2][2];
  __device__ __forceinline__ void load(const void* x, int64_t ldx, int M, int K, int m, int k0, bool xvec) {
    float t[16];
    load8_f32<XT_F32>(x, ldx, M, K, m, k0, xvec, t);
    load8_f32<XT_F32>(x, ldx, M, K, m, k0 + 8, xvec, t + 8);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      __bf16 h, l;
      split_bf16(t[j], h, l);
      v[0][0][j] = h;
      v[0][1][j] = l;
      split_bf16(t[8 + j], h, l);
      v[1][0][j] = h;
      v[1][1][j] = l;
    }
  }
};

// Weight fragment conversion + MFMA for one 16x64 tile against one activation
// fragment.
template <int XT>
struct TileMma {
  static __device__ __forceinline__ void run(u32x4 w, const XFrag<XT>& xf, f32x4& acc);
};

template <>
__device__ __forceinline__ void TileMma<XT_F16>::run(u32x4 w, const XFrag<XT_F16>& xf, f32x4& acc) {
  f16x8 w0, w1;
  u8x16_to_f16(w, w0, w1);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(w0, xf.v[0][0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(w1, xf.v[1][0], acc, 0, 0, 0);
}

template <>
__device__ __forceinline__ void TileMma<XT_BF16>::run(u32x4 w, const XFrag<XT_BF16>& xf, f32x4& acc) {
  bf16x8 w0, w1;
  u8x16_to_bf16(w, w0, w1);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0, xf.v[0][0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1, xf.v[1][0], acc, 0, 0, 0);
}

template <>
__device__ __forceinline__ void TileMma<XT_F32>::run(u32x4 w, const XFrag<XT_F32>& xf, f32x4& acc) {
  bf16x8 w0, w1;
  u8x16_to_bf16(w, w0, w1);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0, xf.v[0][1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1, xf.v[1][1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0, xf.v[0][0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1, xf.v[1][0], acc, 0, 0, 0);
}

__device__ __forceinline__ u32x4 load_tile_nt(const uint8_t* p) {
  return __builtin_nontemporal_load((const u32x4*)p);
}

// ---------------------------------------------------------------------------
// Weight-only
// ---------------------------------------------------------------------------
template <int XT, int G, int MT>
__global__ __launch_bounds__(1024) void gemv_w8_kernel(const void* __restrict__ x, int64_t ldx, int M, int K,
                                                       int Kc, const uint8_t* __restrict__ packed,
                                                       const float* __restrict__ scale,
                                                       const float* __restrict__ bias, int N, int Nt,
                                                       void* __restrict__ y, int yt, int64_t ldy, int flags) {
  extern __shared__ f32x4 red[];  // [waves][G*MT][64]
  const bool xvec = flags & 1;
  const int nw = blockDim.x >> 6;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const int nt0 = blockIdx.x * G;
  const int per = (Kc + nw - 1) / nw;
  const int kb = wave * per;
  const int ke = min(Kc, kb + per);

  f32x4 acc[G][MT];
#pragma unroll
  for (int t = 0; t < G; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const uint8_t* tp[G];
#pragma unroll
  for (int t = 0; t < G; ++t) tp[t] = packed + ((int64_t)(nt0 + t) * Kc) * 1024 + lane * 16;

  for (int kc = kb; kc < ke; ++kc) {
    u32x4 w[G];
#pragma unroll
    for (int t = 0; t < G; ++t) {
      if (nt0 + t < Nt) w[t] = load_tile_nt(tp[t] + (int64_t)kc * 1024);
    }
    XFrag<XT> xf[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xf[mt].load(x, ldx, M, K, mt * 16 + r, kc * 64 + g * 16, xvec);
#pragma unroll
    for (int t = 0; t < G; ++t) {
      if (nt0 + t < Nt) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) TileMma<XT>::run(w[t], xf[mt], acc[t][mt]);
      }
    }
  }

#pragma unroll
  for (int t = 0; t < G; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[(wave * G * MT + t * MT + mt) * 64 + lane] = acc[t][mt];
  __syncthreads();

  const bool yvec_ok = flags & 2;
  for (int p = threadIdx.x; p < G * MT * 64; p += blockDim.x) {
    const int l = p & 63, tm = p >> 6;
    const int t = tm / MT, mt = tm % MT;
    const int m = mt * 16 + (l & 15);
    const int nt = nt0 + t;
    if (m >= M || nt >= Nt) continue;
    f32x4 s = red[tm * 64 + l];
    for (int w = 1; w < nw; ++w) s += red[(w * G * MT + tm) * 64 + l];
    const int n = nt * 16 + (l >> 4) * 4;
    if (n >= N) continue;
    const int nvalid = min(4, N - n);
    f32x4 o;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int nn = min(n + v, N - 1);
      float out = s[v] * scale[nn];
      if (bias) out = out + bias[nn];
      o[v] = out;
    }
    store_y4(y, yt, (int64_t)m * ldy + n, o, yvec_ok && nvalid == 4, nvalid);
  }
}

// ---------------------------------------------------------------------------
// W8A8: activations quantized on the fly with the per-tensor parameters,
// i8 MFMA 16x16x64 with exact int32 accumulation.
// ---------------------------------------------------------------------------
template <int XT>
__device__ __forceinline__ i32x4 load_xq16(const void* x, int64_t ldx, int M, int K, int m, int k0, bool xvec,
                                           float inv, float zpf) {
  float t[16];
  load8_f32<XT>(x, ldx, M, K, m, k0, xvec, t);
  load8_f32<XT>(x, ldx, M, K, m, k0 + 8, xvec, t + 8);
  uint32_t d[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int jj = 4 * i + j;
      const bool valid = m < M && k0 + jj < K;
      const int qv = valid ? quant_act_s8(t[jj], inv, zpf) : 0;
      word |= ((uint32_t)qv & 0xffu) << (8 * j);
    }
    d[i] = word;
  }
  return (i32x4){(int)d[0], (int)d[1], (int)d[2], (int)d[3]};
}

__device__ __forceinline__ i32x4 tile_to_s8(u32x4 w) {
  return (i32x4){(int)(w.x ^ 0x80808080u), (int)(w.y ^ 0x80808080u), (int)(w.z ^ 0x80808080u),
                 (int)(w.w ^ 0x80808080u)};
}

template <int XT, int G, int MT>
__global__ __launch_bounds__(1024) void gemv_w8a8_kernel(const void* __restrict__ x, int64_t ldx, int M, int K,
                                                         int Kc, const uint8_t* __restrict__ packed,
                                                         const float* __restrict__ scale,
                                                         const int32_t* __restrict__ colsum,
                                                         const float* __restrict__ bias, int N, int Nt,
                                                         void* __restrict__ y, int yt, int64_t ldy,
                                                         int32_t* __restrict__ acc_out,
                                                         const float2* __restrict__ partials, int nparts,
                                                         int flags) {
  const bool xvec = flags & 1;
  extern __shared__ i32x4 redi[];  // [waves][G*MT][64]
  __shared__ float qred[32];
  const ActQParams qp = block_qparams_from_partials(partials, nparts, qred);
  const int nw = blockDim.x >> 6;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const int nt0 = blockIdx.x * G;
  const int per = (Kc + nw - 1) / nw;
  const int kb = wave * per;
  const int ke = min(Kc, kb + per);

  i32x4 acc[G][MT];
#pragma unroll
  for (int t = 0; t < G; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = (i32x4){0, 0, 0, 0};

  const uint8_t* tp[G];
#pragma unroll
  for (int t = 0; t < G; ++t) tp[t] = packed + ((int64_t)(nt0 + t) * Kc) * 1024 + lane * 16;

  for (int kc = kb; kc < ke; ++kc) {
    u32x4 w[G];
#pragma unroll
    for (int t = 0; t < G; ++t) {
      if (nt0 + t < Nt) w[t] = load_tile_nt(tp[t] + (int64_t)kc * 1024);
    }
    i32x4 xq[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      xq[mt] = load_xq16<XT>(x, ldx, M, K, mt * 16 + r, kc * 64 + g * 16, xvec, qp.inv, qp.zpf);
#pragma unroll
    for (int t = 0; t < G; ++t) {
      if (nt0 + t < Nt) {
        const i32x4 ws = tile_to_s8(w[t]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[t][mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ws, xq[mt], acc[t][mt], 0, 0, 0);
      }
    }
  }

#pragma unroll
  for (int t = 0; t < G; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) redi[(wave * G * MT + t * MT + mt) * 64 + lane] = acc[t][mt];
  __syncthreads();

  const bool yvec_ok = flags & 2;
  const int corr = 128 - qp.zp;
  for (int p = threadIdx.x; p < G * MT * 64; p += blockDim.x) {
    const int l = p & 63, tm = p >> 6;
    const int t = tm / MT, mt = tm % MT;
    const int m = mt * 16 + (l & 15);
    const int nt = nt0 + t;
    if (m >= M || nt >= Nt) continue;
    i32x4 s = redi[tm * 64 + l];
    for (int w = 1; w < nw; ++w) s += redi[(w * G * MT + tm) * 64 + l];
    const int n = nt * 16 + (l >> 4) * 4;
    if (n >= N) continue;
    const int nvalid = min(4, N - n);
    f32x4 o;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int nn = min(n + v, N - 1);
      const int a = s[v] + corr * colsum[nn];
      if (acc_out && v < nvalid) acc_out[(int64_t)m * N + n + v] = a;
      const float mult = qp.scale * scale[nn];
      o[v] = bias ? __builtin_fmaf((float)a, mult, bias[nn]) : (float)a * mult;
    }
    store_y4(y, yt, (int64_t)m * ldy + n, o, yvec_ok && nvalid == 4, nvalid);
  }
}

// ---------------------------------------------------------------------------
// launch configuration
// ---------------------------------------------------------------------------
struct GemvCfg {
  int g, mt, waves;
};

static GemvCfg pick_gemv(int64_t M, int64_t Nt, int64_t Kc) {
  GemvCfg c;
  c.mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  // K split: 4..16 tiles per wave
  if (Kc >= 128) c.waves = 16;
  else if (Kc >= 32) c.waves = 8;
  else if (Kc >= 8) c.waves = 4;
  else if (Kc >= 2) c.waves = 2;
  else c.waves = 1;
  c.g = 1;
  if (c.mt == 1) {
    while (c.g < 4 && (Nt / (2 * c.g)) * c.waves >= 4096) c.g *= 2;
  }
  return c;
}

template <int XT, int G, int MT>
static void launch_w8_inst(dim3 grid, dim3 block, size_t lds, hipStream_t st, const void* x, int64_t ldx, int M,
                           int K, int Kc, const uint8_t* packed, const float* scale, const float* bias, int N, int Nt,
                           void* y, int yt, int64_t ldy, int flags) {
  hipLaunchKernelGGL((gemv_w8_kernel<XT, G, MT>), grid, block, lds, st, x, ldx, M, K, Kc, packed, scale, bias, N,
                     Nt, y, yt, ldy, flags);
}

template <int XT>
static int launch_w8_xt(const GemvCfg& c, hipStream_t st, const void* x, int64_t ldx, int M, int K, int Kc,
                        const uint8_t* packed, const float* scale, const float* bias, int N, int Nt, void* y, int yt,
                        int64_t ldy, int flags) {
  dim3 grid((unsigned)((Nt + c.g - 1) / c.g)), block(64 * c.waves);
  const size_t lds = (size_t)c.waves * c.g * c.mt * 64 * sizeof(f32x4);
#define SBQ_W8_CASE(G_, MT_)                                                                               \
  if (c.g == G_ && c.mt == MT_) {                                                                          \
    launch_w8_inst<XT, G_, MT_>(grid, block, lds, st, x, ldx, M, K, Kc, packed, scale, bias, N, Nt, y, yt, \
                                ldy, flags);                                                               \
    return check_launch();                                                                                 \
  }
  SBQ_W8_CASE(1, 1)
  SBQ_W8_CASE(2, 1)
  SBQ_W8_CASE(4, 1)
  SBQ_W8_CASE(1, 2)
  SBQ_W8_CASE(1, 4)
#undef SBQ_W8_CASE
  return -1;
}

int launch_gemv_w8(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec, const uint8_t* packed,
                   const float* scale, const float* bias, int64_t N, void* y, int yt, int64_t ldy, hipStream_t st,
                   bool yvec) {
  const int64_t Nt = (N + 15) / 16, Kc = (K + 63) / 64;
  const int xvec_i = (xvec ? 1 : 0) | (yvec ? 2 : 0);
  const GemvCfg c = pick_gemv(M, Nt, Kc);
  switch (xt) {
    case XT_F16: return launch_w8_xt<XT_F16>(c, st, x, ldx, (int)M, (int)K, (int)Kc, packed, scale, bias, (int)N, (int)Nt, y, yt, ldy, xvec_i);
    case XT_BF16: return launch_w8_xt<XT_BF16>(c, st, x, ldx, (int)M, (int)K, (int)Kc, packed, scale, bias, (int)N, (int)Nt, y, yt, ldy, xvec_i);
    case XT_F32: return launch_w8_xt<XT_F32>(c, st, x, ldx, (int)M, (int)K, (int)Kc, packed, scale, bias, (int)N, (int)Nt, y, yt, ldy, xvec_i);
  }
  return -2;
}

template <int XT, int G, int MT>
static void launch_w8a8_inst(dim3 grid, dim3 block, size_t lds, hipStream_t st, const void* x, int64_t ldx, int M,
                             int K, int Kc, const uint8_t* packed, const float* scale, const int32_t* colsum,
                             const float* bias, int N, int Nt, void* y, int yt, int64_t ldy, int32_t* acc_out,
                             const float2* partials, int nparts, int flags) {
  hipLaunchKernelGGL((gemv_w8a8_kernel<XT, G, MT>), grid, block, lds, st, x, ldx, M, K, Kc, packed, scale, colsum,
                     bias, N, Nt, y, yt, ldy, acc_out, partials, nparts, flags);
}

template <int XT>
static int launch_w8a8_xt(const GemvCfg& c, hipStream_t st, const void* x, int64_t ldx, int M, int K, int Kc,
                          const uint8_t* packed, const float* scale, const int32_t* colsum, const float* bias, int N,
                          int Nt, void* y, int yt, int64_t ldy, int32_t* acc_out, const float2* partials, int nparts,
                          int flags) {
  dim3 grid((unsigned)((Nt + c.g - 1) / c.g)), block(64 * c.waves);
  const size_t lds = (size_t)c.waves * c.g * c.mt * 64 * sizeof(i32x4);
#define SBQ_W8A8_CASE(G_, MT_)                                                                                 \
  if (c.g == G_ && c.mt == MT_) {                                                                              \
    launch_w8a8_inst<XT, G_, MT_>(grid, block, lds, st, x, ldx, M, K, Kc, packed, scale, colsum, bias, N, Nt, \
                                  y, yt, ldy, acc_out, partials, nparts, flags);                               \
    return check_launch();                                                                                     \
  }
  SBQ_W8A8_CASE(1, 1)
  SBQ_W8A8_CASE(2, 1)
  SBQ_W8A8_CASE(4, 1)
  SBQ_W8A8_CASE(1, 2)
  SBQ_W8A8_CASE(1, 4)
#undef SBQ_W8A8_CASE
  return -1;
}

int launch_gemv_w8a8(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec, const uint8_t* packed,
                     const float* scale, const int32_t* colsum, const float* bias, int64_t N, void* y, int yt,
                     int64_t ldy, int32_t* acc_out, const float2* partials, int nparts, hipStream_t st,
                     bool yvec) {
  const int64_t Nt = (N + 15) / 16, Kc = (K + 63) / 64;
  const int xvec_i = (xvec ? 1 : 0) | (yvec ? 2 : 0);
  const GemvCfg c = pick_gemv(M, Nt, Kc);
  switch (xt) {
    case XT_F16: return launch_w8a8_xt<XT_F16>(c, st, x, ldx, (int)M, (int)K, (int)Kc, packed, scale, colsum, bias, (int)N, (int)Nt, y, yt, ldy, acc_out, partials, nparts, xvec_i);
    case XT_BF16: return launch_w8a8_xt<XT_BF16>(c, st, x, ldx, (int)M, (int)K, (int)Kc, packed, scale, colsum, bias, (int)N, (int)Nt, y, yt, ldy, acc_out, partials, nparts, xvec_i);
    case XT_F32: return launch_w8a8_xt<XT_F32>(c, st, x, ldx, (int)M, (int)K, (int)Kc, packed, scale, colsum, bias, (int)N, (int)Nt, y, yt, ldy, acc_out, partials, nparts, xvec_i);
  }
  return -2;
}

}  // namespace sbq

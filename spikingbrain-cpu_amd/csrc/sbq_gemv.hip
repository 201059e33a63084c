// sbq_gemv.hip - decode (small-M) quantized linear, HBM-bandwidth bound.
//
// Replaces the per-token projections of spikingbrain_cpu/quant.py:41-53
// (Int8Linear.forward, weight-only) and quant.py:63-66 (DynamicInt8Linear,
// W8A8) at the decode shapes the engine issues (engine.py:106: M = 1).
//
// Work decomposition: a workgroup owns G consecutive 16-row weight tiles and
// splits K over its (up to 16) waves, P 64-wide K tiles per wave.  A wave
// issues every one of its G*P 1 KiB tile loads (16 bytes per lane,
// non-temporal) before it consumes any, so a kernel has its whole working set
// in flight at once instead of one round trip per K step.  The activation
// fragments are loaded before the weights: loads retire in order, so waiting
// for them never waits for the weight stream.  Tiles are converted in
// registers and fed to MFMA 16x16 instructions with the activation fragment
// as the second operand.  Per-wave partial tiles are summed in LDS in a fixed
// wave order (deterministic), then scale/bias are applied and each lane stores
// four consecutive outputs as one vector.
#include <algorithm>
#include <type_traits>

#include "sbq_common.h"
#include "sbq_gemv_ops.h"
#include "sbq_launch.h"

namespace sbq {

// ---------------------------------------------------------------------------
// Persistent streaming kernel (weight-only and W8A8).
//
// A workgroup of `waves` waves owns a fixed K split: wave w always covers K
// tiles [w*P, w*P + P).  Groups of G weight tiles are assigned round-robin
// (group = blockIdx.x + i * gridDim.x).  The weight tiles of the next NB-1
// groups (and their scale/bias/colsum values) are in flight while the current
// group is multiplied, reduced across waves in LDS and stored.
//
// Activation modes (XM):
//   XM_REG   each wave loads the fragments of its K split once, into registers
//   XM_LDS   the workgroup stages x[M][K] in LDS once; fragments are read on use
//   XM_CHUNK fragments are re-read from global memory (L2) per group, XC K tiles
//            at a time (for x too large for LDS; used with NB = 1)
// In every mode the first activation loads are issued before the weight loads:
// loads retire in order, so waiting for them never waits for the weights.
// ---------------------------------------------------------------------------
enum XMode { XM_REG = 0, XM_LDS = 1, XM_CHUNK = 2 };


// Per-thread epilogue operands of one group: thread t < G*MT*64 finishes pair
// (tile t/64/MT, token tile (t/64)%MT, lane t%64), i.e. outputs n..n+3 of row m.
struct EpiVals {
  f32x4 sc, bi;
  i32x4 cs;
};

template <int G, int MT, bool W8A8>
__device__ __forceinline__ void load_epi(const GemvArgs& a, int grp, EpiVals& e) {
  const int p = threadIdx.x;
  if (p >= G * MT * 64 || grp >= a.ngroups) return;
  const int l = p & 63, t = (p >> 6) / MT;
  const int n = (grp * G + t) * 16 + (l >> 4) * 4;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int nn = min(n + v, a.N - 1);
    e.sc[v] = a.scale[nn];
    e.bi[v] = a.bias ? a.bias[nn] : 0.0f;
    if constexpr (W8A8) e.cs[v] = a.colsum[nn];
  }
}

template <int G, int P>
__device__ __forceinline__ void load_w(const GemvArgs& a, int grp, int kb, int lane, u32x4 (&w)[G][P]) {
  if (grp >= a.ngroups) return;
#pragma unroll
  for (int t = 0; t < G; ++t)
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int nt = grp * G + t;
      if (nt < a.Nt && kb + p < a.Kc) w[t][p] = load_tile_nt(a.packed + ((int64_t)nt * a.Kc + kb + p) * 1024 + lane * 16);
    }
}

// Activation fragments of K tiles [kb+p0, kb+p0+CNT) from global memory.
template <int XT, int MT, int CNT>
__device__ __forceinline__ void load_x_frags(const GemvArgs& a, int kb, int p0, int pend, int lane,
                                             XRaw<XT> (&xr)[CNT][MT]) {
  const int r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int p = 0; p < CNT; ++p)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      if (p0 + p < pend && kb + p0 + p < a.Kc)
        xr[p][mt].load(a.x, a.ldx, a.M, a.K, mt * 16 + r, (kb + p0 + p) * 64 + g * 16, a.flags & 1);
}

// Multiply-accumulate one K tile of every weight tile of the group.
template <int XT, int MT, int G, bool W8A8, typename Acc>
__device__ __forceinline__ void mma_ktile(const u32x4 (&wk)[G], const XRaw<XT> (&xf)[MT], const i32x4* xq,
                                          int nt0, int Nt, const GemvArgs& a, int lane, int k0, const ActQParams& qp,
                                          Acc (&acc)[G][MT]) {
#pragma unroll
  for (int t = 0; t < G; ++t) {
    if (nt0 + t >= Nt) continue;
    if constexpr (W8A8) {
      const i32x4 ws = tile_to_s8(wk[t]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const i32x4 q = xq ? xq[mt] : quant_frag<XT>(xf[mt], a.M, a.K, mt * 16 + (lane & 15), k0, qp.inv, qp.zpf);
        acc[t][mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ws, q, acc[t][mt], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) tile_mma<XT>(wk[t], xf[mt], acc[t][mt]);
    }
  }
}

// Cross-wave reduction of the group in LDS (fixed wave order), epilogue and
// vector store of four outputs per lane.
template <int G, int MT, bool W8A8, typename Acc>
__device__ __forceinline__ void reduce_store(const GemvArgs& a, int grp, int lane, const Acc (&acc)[G][MT],
                                             const EpiVals& e, const ActQParams& qp, void* red) {
  const int wave = threadIdx.x >> 6;
  const int nt0 = grp * G;
  Acc* redv = (Acc*)red;
#pragma unroll
  for (int t = 0; t < G; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) redv[(wave * G * MT + t * MT + mt) * 64 + lane] = acc[t][mt];
  __syncthreads();

  const int pidx = threadIdx.x;
  if (pidx < G * MT * 64) {
    const int nw = blockDim.x >> 6;
    const int l = pidx & 63, tm = pidx >> 6;
    const int t = tm / MT, mt = tm % MT;
    const int m = mt * 16 + (l & 15);
    const int nt = nt0 + t;
    const int n = nt * 16 + (l >> 4) * 4;
    if (m < a.M && nt < a.Nt && n < a.N) {
      Acc s = redv[tm * 64 + l];
      for (int ww = 1; ww < nw; ++ww) s += redv[(ww * G * MT + tm) * 64 + l];
      const int nvalid = min(4, a.N - n);
      f32x4 o;
      if constexpr (W8A8) {
        const int corr = 128 - qp.zp;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int av = s[v] + corr * e.cs[v];
          if (a.acc_out && v < nvalid) a.acc_out[(int64_t)m * a.N + n + v] = av;
          const float mult = qp.scale * e.sc[v];
          o[v] = a.bias ? __builtin_fmaf((float)av, mult, e.bi[v]) : (float)av * mult;
        }
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float out = s[v] * e.sc[v];
          if (a.bias) out = out + e.bi[v];
          o[v] = out;
        }
      }
      store_y4(a.y, a.yt, (int64_t)m * a.ldy + n, o, (a.flags & 2) && nvalid == 4, nvalid);
    }
  }
  __syncthreads();  // the next group reuses the reduction buffer
}

template <int XT, int MT, int G, int P, bool W8A8, int XM, int XR, int XC>
__device__ __forceinline__ void process_group(const GemvArgs& a, int grp, int kb, int lane,
                                              const u32x4 (&w)[G][P], XRaw<XT> (&xr)[XR][MT],
                                              const i32x4 (&xq)[XM == XM_REG ? P : 1][MT], const EpiVals& e,
                                              const ActQParams& qp, void* red, const uint8_t* xl, int Kp) {
  typedef typename std::conditional<W8A8, i32x4, f32x4>::type Acc;
  const int r = lane & 15, g = lane >> 4;
  const int nt0 = grp * G;
  Acc acc[G][MT];
#pragma unroll
  for (int t = 0; t < G; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = Acc{0, 0, 0, 0};

#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int kc = kb + p;
    if (kc >= a.Kc) continue;
    // LDS / chunked activations: keep the per-tile activation reads next to
    // their use (hoisting all of them would exceed the register budget)
    if constexpr (XM != XM_REG) {
      if (p > 0) __builtin_amdgcn_sched_barrier(0);
    }
    u32x4 wk[G];
#pragma unroll
    for (int t = 0; t < G; ++t) wk[t] = w[t][p];
    if constexpr (XM == XM_REG) {
      mma_ktile<XT, MT, G, W8A8>(wk, xr[p], W8A8 ? xq[p] : nullptr, nt0, a.Nt, a, lane, kc * 64 + g * 16, qp, acc);
    } else if constexpr (XM == XM_LDS) {
      XRaw<XT> xf[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xf[mt].load_lds(xl, Kp, a.M, mt * 16 + r, kc * 64 + g * 16);
      mma_ktile<XT, MT, G, W8A8>(wk, xf, nullptr, nt0, a.Nt, a, lane, kc * 64 + g * 16, qp, acc);
    }
  }
  reduce_store<G, MT, W8A8>(a, grp, lane, acc, e, qp, red);
}

// XM_CHUNK: the wave's P K tiles run as a pipeline of XC-tile sub-chunks; the
// activations (re-read from L2 per group) and weight tiles of sub-chunk c+1
// are loaded while sub-chunk c is multiplied.
template <int XT, int MT, int G, int P, bool W8A8, int XC>
__device__ __forceinline__ void process_group_chunked(const GemvArgs& a, int grp, int kb, int lane,
                                                      const EpiVals& e, const ActQParams& qp, void* red) {
  typedef typename std::conditional<W8A8, i32x4, f32x4>::type Acc;
  constexpr int NCH = (P + XC - 1) / XC;
  const int g = lane >> 4;
  const int nt0 = grp * G;
  XRaw<XT> xc[2][XC][MT];
  u32x4 wc[2][G][XC];
  auto load_chunk = [&](int c, int b) {
    load_x_frags<XT, MT, XC>(a, kb, c * XC, P, lane, xc[b]);
#pragma unroll
    for (int t = 0; t < G; ++t)
#pragma unroll
      for (int j = 0; j < XC; ++j) {
        const int p = c * XC + j, nt = nt0 + t;
        if (p < P && nt < a.Nt && kb + p < a.Kc)
          wc[b][t][j] = load_tile_nt(a.packed + ((int64_t)nt * a.Kc + kb + p) * 1024 + lane * 16);
      }
  };
  Acc acc[G][MT];
#pragma unroll
  for (int t = 0; t < G; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = Acc{0, 0, 0, 0};
  load_chunk(0, 0);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (c + 1 < NCH) load_chunk(c + 1, (c + 1) & 1);
#pragma unroll
    for (int j = 0; j < XC; ++j) {
      const int p = c * XC + j, kc = kb + p;
      if (p >= P || kc >= a.Kc) continue;
      u32x4 wk[G];
#pragma unroll
      for (int t = 0; t < G; ++t) wk[t] = wc[c & 1][t][j];
      mma_ktile<XT, MT, G, W8A8>(wk, xc[c & 1][j], nullptr, nt0, a.Nt, a, lane, kc * 64 + g * 16, qp, acc);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  reduce_store<G, MT, W8A8>(a, grp, lane, acc, e, qp, red);
}

template <int XT, int MT, int G, int P, bool W8A8, int XM, int NB, int SC = kStageChunks>
__global__ __launch_bounds__(1024) void gemv_kernel(const GemvArgs a) {
  // dynamic LDS: [waves][G*MT][64] accumulators (the head doubles as qparams
  // scratch), then with XM_LDS the activations x[M][Kp] (zero padded)
  extern __shared__ f32x4 red[];
  constexpr int XC = XT == XT_F32 ? 1 : 2;                           // XM_CHUNK sub-chunk (K tiles)
  constexpr int XR = XM == XM_REG ? P : 1;
  constexpr int XSZ = x_bytes<XT>();
  static_assert(XM != XM_CHUNK || NB == 1, "chunked activations reload per group: one weight buffer");
  const int nw = blockDim.x >> 6;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kb = wave * P;
  const int Kp = a.Kc * 64;
  uint8_t* xl = (uint8_t*)(red + nw * G * MT * 64);
  int grp = blockIdx.x;

  // W8A8: activation min/max partials first (nparts <= 256, blockDim.x >= 64)
  float2 part[4];
  if constexpr (W8A8) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = threadIdx.x + i * blockDim.x;
      part[i] = idx < a.nparts ? a.partials[idx] : make_float2(0.0f, 0.0f);
    }
  }
  XRaw<XT> xr[XR][MT];
  u32x4 stg[XM == XM_LDS ? SC : 1];
  const int row_chunks = Kp * XSZ / 16;
  if constexpr (XM == XM_LDS) {
#pragma unroll
    for (int i = 0; i < SC; ++i) {
      const int c = threadIdx.x + i * blockDim.x;
      if (c < a.M * row_chunks) {
        const int m = c / row_chunks;
        const int k0 = (c - m * row_chunks) * (16 / XSZ);
        const uint8_t* src = (const uint8_t*)a.x + ((int64_t)m * a.ldx + k0) * XSZ;
        if ((a.flags & 1) && k0 + 16 / XSZ <= a.K) {
          stg[i] = *(const u32x4*)src;
        } else {
          uint8_t b[16];
#pragma unroll
          for (int j = 0; j < 16; ++j) b[j] = (k0 + j / XSZ < a.K) ? src[j] : (uint8_t)0;
          stg[i] = __builtin_bit_cast(u32x4, b);
        }
      }
    }
  } else if constexpr (XM == XM_REG) {
    load_x_frags<XT, MT, XR>(a, kb, 0, P, lane, xr);
  }

  // weight ring (the chunked mode keeps its own sub-chunk buffers)
  constexpr int WP = XM == XM_CHUNK ? 1 : P;
  u32x4 wbuf[NB][G][WP];
  EpiVals ebuf[NB];
  if constexpr (XM != XM_CHUNK) {
#pragma unroll
    for (int b = 0; b < (NB > 1 ? NB - 1 : 1); ++b) {
      load_w<G, P>(a, grp + b * (int)gridDim.x, kb, lane, wbuf[b]);
      load_epi<G, MT, W8A8>(a, grp + b * (int)gridDim.x, ebuf[b]);
    }
  } else {
    load_epi<G, MT, W8A8>(a, grp, ebuf[0]);
  }

  if constexpr (XM == XM_LDS) {
#pragma unroll
    for (int i = 0; i < SC; ++i) {
      const int c = threadIdx.x + i * blockDim.x;
      if (c < a.M * row_chunks) *(u32x4*)(xl + (int64_t)c * 16) = stg[i];
    }
    __syncthreads();
  }

  ActQParams qp{};
  i32x4 xq[XM == XM_REG ? P : 1][MT];
  if constexpr (W8A8) {
    float mn = 0.0f, mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mn = fminf(mn, part[i].x);
      mx = fmaxf(mx, part[i].y);
    }
    float* qred = (float*)red;
    mn = wave_min(mn);
    mx = wave_max(mx);
    if (lane == 0) {
      qred[2 * wave] = mn;
      qred[2 * wave + 1] = mx;
    }
    __syncthreads();
    mn = qred[0];
    mx = qred[1];
    for (int i = 1; i < nw; ++i) {
      mn = fminf(mn, qred[2 * i]);
      mx = fmaxf(mx, qred[2 * i + 1]);
    }
    __syncthreads();
    qp = choose_act_qparams(mn, mx);
    if constexpr (XM == XM_REG) {
      const int r = lane & 15, g = lane >> 4;
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          xq[p][mt] = quant_frag<XT>(xr[p][mt], a.M, a.K, mt * 16 + r, (kb + p) * 64 + g * 16, qp.inv, qp.zpf);
    }
  }

  if constexpr (XM == XM_CHUNK) {
    while (true) {
      process_group_chunked<XT, MT, G, P, W8A8, XC>(a, grp, kb, lane, ebuf[0], qp, red);
      grp += gridDim.x;
      if (grp >= a.ngroups) break;
      load_epi<G, MT, W8A8>(a, grp, ebuf[0]);
    }
  } else if constexpr (NB == 1) {
    while (true) {
      process_group<XT, MT, G, P, W8A8, XM, XR, XC>(a, grp, kb, lane, wbuf[0], xr, xq, ebuf[0], qp, red, xl, Kp);
      grp += gridDim.x;
      if (grp >= a.ngroups) break;
      load_w<G, P>(a, grp, kb, lane, wbuf[0]);
      load_epi<G, MT, W8A8>(a, grp, ebuf[0]);
    }
  } else {
    // ring: buffer b holds group grp; the load NB-1 groups ahead goes into the
    // buffer the previous group just released
    while (true) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int ahead = grp + (NB - 1) * (int)gridDim.x;
        load_w<G, P>(a, ahead, kb, lane, wbuf[(b + NB - 1) % NB]);
        load_epi<G, MT, W8A8>(a, ahead, ebuf[(b + NB - 1) % NB]);
        if (grp >= a.ngroups) return;
        process_group<XT, MT, G, P, W8A8, XM, XR, XC>(a, grp, kb, lane, wbuf[b], xr, xq, ebuf[b], qp, red, xl, Kp);
        grp += gridDim.x;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// launch configuration
// ---------------------------------------------------------------------------
struct GemvCfg {
  int mt, g, p, waves, xm, nb, sc;
  bool ok;
};

// Measured on MI355X (M = 1, fp16, 4096..151936 x 4096..12288): one-shot
// workgroups (grid = #groups, no persistence, NB = 1) with 8 KiB of weight
// tiles per wave beat persistent rings: independent workgroups overlap on the
// CU by themselves.  P = 8 K tiles per wave (8 waves at K = 4096), P = 12 for
// K up to 12288, P = Kc below 8.  Activations: staged in LDS with SC 16-byte
// chunks per thread when x[M][K] allows SC <= 4; otherwise registers
// (short K splits) or per-group chunks.  Every instance below fits the
// register budget of its workgroup without spilling.
static GemvCfg pick_gemv(int64_t M, int64_t Nt, int64_t Kc, bool w8a8, int xt) {
  (void)Nt;
  GemvCfg c{};
  if (M > 32 || Kc > 192) return c;
  c.mt = M <= 16 ? 1 : 2;
  c.p = Kc <= 8 ? (Kc <= 1 ? 1 : (Kc <= 2 ? 2 : (Kc <= 4 ? 4 : 8))) : (Kc <= 128 ? 8 : 12);
  c.waves = (int)((Kc + c.p - 1) / c.p);
  c.g = 1;
  c.nb = 1;
  c.ok = true;
  const int64_t xbytes = M * Kc * 64 * (xt == XT_F32 ? 4 : 2);
  const int64_t per_thread = (xbytes + 16 * 64 * c.waves - 1) / (16 * 64 * c.waves);
  if (c.mt == 1 && per_thread <= 4) {
    c.xm = XM_LDS;
    c.sc = per_thread <= 1 ? 1 : (per_thread <= 2 ? 2 : 4);
    return c;
  }
  c.sc = 1;
  const int reg_p = xt == XT_F32 ? 1 : (w8a8 ? 2 : 4);
  if (c.p > reg_p && Kc <= 16 * reg_p) {  // a shorter K split keeps x in registers
    c.p = reg_p;
    c.waves = (int)((Kc + c.p - 1) / c.p);
  }
  if (c.p <= reg_p) {
    c.xm = XM_REG;
    // the epilogue takes one thread per output pair (G * MT * 64 threads):
    // two row tiles of x need two waves even when one wave covers K (the
    // second wave's K range is empty and adds zeros)
    if (c.waves < c.mt) c.waves = c.mt;
  } else if (c.mt == 1) {
    c.xm = XM_CHUNK;
  } else {
    c.ok = false;
  }
  return c;
}

bool gemv_supports(int64_t M, int64_t K, bool w8a8, int xt) {
  if (M < 1) return false;
  return pick_gemv(M, 1, (K + 63) / 64, w8a8, xt).ok;
}

// Forward declaration: the instance table below decides whether a picked
// configuration has a kernel.
static bool gemv_instance_exists(const GemvCfg& c, int xt, bool w8a8);

int gemv_config_info(int64_t M, int64_t K, bool w8a8, int xt, int32_t* info) {
  const int64_t Kc = (K + 63) / 64;
  const GemvCfg c = pick_gemv(M, 1, Kc, w8a8, xt);
  const int64_t xb = xt == XT_F32 ? 4 : 2;
  const int64_t lds = (int64_t)c.waves * c.g * c.mt * 64 * 16 + (c.xm == XM_LDS ? M * Kc * 64 * xb : 0);
  info[0] = c.ok ? 1 : 0;
  info[1] = c.mt;
  info[2] = c.g;
  info[3] = c.p;
  info[4] = c.waves;
  info[5] = c.xm;
  info[6] = c.sc;
  info[7] = (int32_t)std::min<int64_t>(lds, 0x7fffffff);
  info[8] = c.ok && gemv_instance_exists(c, xt, w8a8) ? 1 : 0;
  return 0;
}

// (MT, P, XM, SC).  Covers every configuration pick_gemv returns: P is one of
// {1, 2, 4, 8, 12}, SC one of {1, 2, 4}; XM_REG only with P <= 4 (MT 1 or 2);
// XM_CHUNK only with P in {8, 12} (K > 16 register-held tiles per wave).
#define SBQ_GEMV_CONFIGS(X) \
  X(1, 1, XM_LDS, 1)        \
  X(1, 1, XM_LDS, 2)        \
  X(1, 1, XM_LDS, 4)        \
  X(1, 2, XM_LDS, 1)        \
  X(1, 2, XM_LDS, 2)        \
  X(1, 2, XM_LDS, 4)        \
  X(1, 4, XM_LDS, 1)        \
  X(1, 4, XM_LDS, 2)        \
  X(1, 4, XM_LDS, 4)        \
  X(1, 8, XM_LDS, 1)        \
  X(1, 8, XM_LDS, 2)        \
  X(1, 8, XM_LDS, 4)        \
  X(1, 12, XM_LDS, 1)       \
  X(1, 12, XM_LDS, 2)       \
  X(1, 12, XM_LDS, 4)       \
  X(1, 1, XM_REG, 1)        \
  X(1, 2, XM_REG, 1)        \
  X(1, 4, XM_REG, 1)        \
  X(1, 8, XM_CHUNK, 1)      \
  X(1, 12, XM_CHUNK, 1)     \
  X(2, 1, XM_REG, 1)        \
  X(2, 2, XM_REG, 1)        \
  X(2, 4, XM_REG, 1)

// Instances pick_gemv can select for an activation type / format.
template <int XT, bool W8A8, int MT, int P, int XM>
constexpr bool gemv_instance_used() {
  if (XM == XM_REG) return P <= (XT == XT_F32 ? 1 : (W8A8 ? 2 : 4));
  if (XM == XM_CHUNK) return MT == 1 && P > (XT == XT_F32 ? 1 : (W8A8 ? 2 : 4));
  return MT == 1;
}

template <int XT, bool W8A8>
static int launch_gemv_xt(const GemvCfg& c, GemvArgs a, hipStream_t st) {
  a.ngroups = (a.Nt + c.g - 1) / c.g;
  size_t lds = (size_t)c.waves * c.g * c.mt * 64 * sizeof(f32x4);
  if (c.xm == XM_LDS) lds += (size_t)a.M * a.Kc * 64 * x_bytes<XT>();
#define SBQ_GEMV_CASE(MT_, P_, XM_, SC_)                                                                   \
  if constexpr (gemv_instance_used<XT, W8A8, MT_, P_, XM_>()) {                                          \
    if (c.mt == MT_ && c.p == P_ && c.xm == XM_ && c.sc == SC_) {                                        \
      hipLaunchKernelGGL((gemv_kernel<XT, MT_, 1, P_, W8A8, XM_, 1, SC_>), dim3(a.ngroups), dim3(64 * c.waves), \
                         lds, st, a);                                                                    \
      return check_launch();                                                                             \
    }                                                                                                    \
  }
  SBQ_GEMV_CONFIGS(SBQ_GEMV_CASE)
#undef SBQ_GEMV_CASE
  return -1;
}

template <int XT, bool W8A8>
static bool gemv_instance_exists_xt(const GemvCfg& c) {
#define SBQ_GEMV_HAS(MT_, P_, XM_, SC_)                                                   \
  if constexpr (gemv_instance_used<XT, W8A8, MT_, P_, XM_>()) {                         \
    if (c.mt == MT_ && c.p == P_ && c.xm == XM_ && c.sc == SC_ && c.g == 1) return true; \
  }
  SBQ_GEMV_CONFIGS(SBQ_GEMV_HAS)
#undef SBQ_GEMV_HAS
  return false;
}

static bool gemv_instance_exists(const GemvCfg& c, int xt, bool w8a8) {
  switch (xt) {
    case XT_F16: return w8a8 ? gemv_instance_exists_xt<XT_F16, true>(c) : gemv_instance_exists_xt<XT_F16, false>(c);
    case XT_BF16: return w8a8 ? gemv_instance_exists_xt<XT_BF16, true>(c) : gemv_instance_exists_xt<XT_BF16, false>(c);
    case XT_F32: return w8a8 ? gemv_instance_exists_xt<XT_F32, true>(c) : gemv_instance_exists_xt<XT_F32, false>(c);
  }
  return false;
}

// The fast-path arguments with the fused greedy token attached when it is
// asked for and applies (fp32 y, M <= 16).
static GemvArgs with_argmax(GemvArgs a, const GemvArgmaxOut* am) {
  if (am && a.yt == XT_F32 && a.M <= 16) {
    a.flags |= kGemvArgmax;
    a.am_state = am->state;
    a.idx = am->idx;
  }
  return a;
}

int launch_gemv_w8(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec, const uint8_t* packed,
                   const float* scale, const float* bias, int64_t N, void* y, int yt, int64_t ldy, hipStream_t st,
                   bool yvec, GemvArgmaxOut* am) {
  const int64_t Nt = (N + 15) / 16, Kc = (K + 63) / 64;
  const GemvCfg c = pick_gemv(M, Nt, Kc, false, xt);
  if (!c.ok) return -1;
  GemvArgs a{};
  a.x = x; a.ldx = ldx; a.M = (int)M; a.K = (int)K; a.Kc = (int)Kc;
  a.packed = packed; a.scale = scale; a.bias = bias;
  a.N = (int)N; a.Nt = (int)Nt; a.y = y; a.yt = yt; a.ldy = ldy;
  a.flags = (xvec ? 1 : 0) | (yvec ? 2 : 0);
  int fid, fks;
  if (pick_gemv_fast(M, K, N, xt, false, xvec, &fid, &fks)) {
    const GemvArgs f = with_argmax(a, am);
    const int rc = launch_gemv_fast_cfg(fid, fks, f, xt, false, st);
    if (rc != -1) {
      if (am) am->fused = rc == 0 && (f.flags & kGemvArgmax);
      return rc;
    }
  }
  switch (xt) {
    case XT_F16: return launch_gemv_xt<XT_F16, false>(c, a, st);
    case XT_BF16: return launch_gemv_xt<XT_BF16, false>(c, a, st);
    case XT_F32: return launch_gemv_xt<XT_F32, false>(c, a, st);
  }
  return -2;
}

// Weight-only decode over several 16-row tiles of x (16 < M <= 64, fp16 /
// bf16 x with aligned rows, 64 | K); -1 when that path does not apply.
int launch_gemv_w8_mt(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec, const uint8_t* packed,
                      const float* scale, const float* bias, int64_t N, void* y, int yt, int64_t ldy, hipStream_t st,
                      bool yvec, bool gemm_alt) {
  GemvArgs a{};
  a.x = x; a.ldx = ldx; a.M = (int)M; a.K = (int)K; a.Kc = (int)((K + 63) / 64);
  a.packed = packed; a.scale = scale; a.bias = bias;
  a.N = (int)N; a.Nt = (int)((N + 15) / 16); a.y = y; a.yt = yt; a.ldy = ldy;
  a.flags = (xvec ? kGemvXVec : 0) | (yvec ? kGemvYVec : 0);
  return launch_gemv_mt(a, xt, st, gemm_alt);
}

// Independent linears of one M, K and dtypes in one fast-path launch (picked
// as one linear of their summed rows): weight-only, or int8-dyn (w8a8: each
// segment's colsum set) with the activation min/max reduced in the kernel.
// -1: the fast path does not apply; the caller runs them one by one.
int launch_gemv_w8_grouped(const GemvSeg* segs, int n, int xt, int64_t M, int64_t K, bool xvec, int yt, bool yvec,
                           hipStream_t st, bool w8a8) {
  if (n < 2 || n > kGemvMaxSeg) return -1;
  int64_t nt = 0;
  for (int i = 0; i < n; ++i) nt += segs[i].Nt;
  int fid, fks;
  if (!pick_gemv_fast(M, K, nt * 16, xt, w8a8, xvec, &fid, &fks)) return -1;
  GemvArgs a{};
  a.M = (int)M; a.K = (int)K; a.Kc = (int)(K / 64);
  a.yt = yt;
  a.flags = (xvec ? kGemvXVec : 0) | (yvec ? kGemvYVec : 0);
  a.nseg = n;
  for (int i = 0; i < n; ++i) a.seg[i] = segs[i];
  return launch_gemv_fast_grouped(fid, fks, a, xt, w8a8, st);
}

int launch_gemv_w8a8(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec, const uint8_t* packed,
                     const float* scale, const int32_t* colsum, const float* bias, int64_t N, void* y, int yt,
                     int64_t ldy, int32_t* acc_out, float2* partials, hipStream_t st, bool yvec,
                     GemvArgmaxOut* am) {
  const int64_t Nt = (N + 15) / 16, Kc = (K + 63) / 64;
  const GemvCfg c = pick_gemv(M, Nt, Kc, true, xt);
  if (!c.ok) return -1;
  GemvArgs a{};
  a.x = x; a.ldx = ldx; a.M = (int)M; a.K = (int)K; a.Kc = (int)Kc;
  a.packed = packed; a.scale = scale; a.bias = bias; a.colsum = colsum;
  a.N = (int)N; a.Nt = (int)Nt; a.y = y; a.yt = yt; a.ldy = ldy; a.acc_out = acc_out;
  a.flags = (xvec ? 1 : 0) | (yvec ? 2 : 0);
  int fid, fks;
  const bool fast = pick_gemv_fast(M, K, N, xt, true, xvec, &fid, &fks);
  if (fast) {  // small x: the kernel reduces the activation min/max itself
    a.nparts = 0;
    const GemvArgs f = with_argmax(a, am);
    const int rc = launch_gemv_fast_cfg(fid, fks, f, xt, true, st);
    if (rc != -1) {
      if (am) am->fused = rc == 0 && (f.flags & kGemvArgmax);
      return rc;
    }
  }
  const int np = minmax_nparts(M, K);
  int rc = launch_minmax_partials(x, xt, M, K, ldx, partials, np, st);
  if (rc) return rc;
  a.partials = partials;
  a.nparts = np;
  if (fast) {
    const GemvArgs f = with_argmax(a, am);
    rc = launch_gemv_fast_cfg(fid, fks, f, xt, true, st);
    if (rc != -1) {
      if (am) am->fused = rc == 0 && (f.flags & kGemvArgmax);
      return rc;
    }
  }
  switch (xt) {
    case XT_F16: return launch_gemv_xt<XT_F16, true>(c, a, st);
    case XT_BF16: return launch_gemv_xt<XT_BF16, true>(c, a, st);
    case XT_F32: return launch_gemv_xt<XT_F32, true>(c, a, st);
  }
  return -2;
}

}  // namespace sbq

// sbq_gemv_fast.hip - decode GEMV for the aligned common case.
//
// Replaces spikingbrain_cpu/quant.py:41-53 (Int8Linear.forward, weight-only)
// and quant.py:63-66 (DynamicInt8Linear.forward, W8A8) at decode shapes when
// M <= 16, K % 64 == 0 and the activation rows are 16-byte aligned - every
// projection of the model (K = 128, 2560, 4096, 9728, 12288).  Other shapes
// take the general kernel in sbq_gemv.hip.
//
// A workgroup of KS waves owns G consecutive 16-row weight tiles.  Wave ks
// covers the K tiles [ks*KW, ks*KW + KW) and streams them D at a time: the D
// (x G) tile loads of the next step are issued right after the tiles of the
// current step are consumed.  Loads are never guarded by branches (indexes are
// clamped instead, and the few surplus tiles of the last step are not
// multiplied), so the compiler's s_waitcnt counting is exact: each tile waits
// for itself only.
//
// Activations, in one of two modes:
//   XL   the workgroup copies x[M][K] into LDS with global_load_lds (16 bytes
//        per lane straight into LDS) before its weight loads, waits for those
//        copies only (vmcnt = number of weight loads issued after them) and
//        reads fragments from LDS on use;
//   direct  each lane loads its 16-element fragment of row min(r, M-1) per
//        tile from global memory (L2-resident) next to the weight tile.
// fp32 x in XL mode (weight-only, M <= 8) is split once, after the copy, into
// bf16 high and remainder planes in LDS; MFMA columns 0..7 multiply the high
// planes, columns 8..15 the remainders, and the epilogue adds the pairs.
// Lanes of rows >= M compute on a duplicate row and never store.
//
// Per-wave partial tiles are summed through LDS in wave order 0..KS-1 by wave
// t for row tile t, then scale / bias (W8A8: zero-point correction and the
// fbgemm requantization) are applied and each lane stores 4 outputs.
// Barriers are s_barrier without __syncthreads()'s fence: the fence would wait
// for every outstanding weight load.
#include <type_traits>

#include "sbq_common.h"
#include "sbq_gemv_ops.h"
#include "sbq_index.h"
#include "sbq_launch.h"

namespace sbq {

namespace {

constexpr int kFastXLdsBytes = 32768;  // x[M][K] copied to LDS up to this size
constexpr int kFastXLdsWideBytes = 81920;  // ... with 5 row tiles per workgroup (one workgroup per CU)
constexpr int kFastMaxWaves = 8;
constexpr int kFusedChunks = 8;         // QM 2: 16-byte chunks of x per thread (at most)
constexpr int kFusedChunksWide = 10;    // ... fp32 x with five row tiles per workgroup (one 512-thread workgroup per CU)
constexpr int kFusedMinWaves = 4;       // W8A8 picks: 256 threads (QM 1: one min/max partial each)
constexpr int kFastSplitBytes = 49152;  // fp32 x split into bf16 planes in LDS up to this size
constexpr int kSplitChunks = 12;        // fp32 x split: 16-byte chunks of x per thread (at most)
constexpr int kSplitRegChunks = 10;     // ... held in registers by five-row-tile workgroups
constexpr int kSplitWideBytes = 81920;  // fp32 x split by five-row-tile workgroups up to this size

__device__ __forceinline__ void lds_copy16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// LDS writes of this wave complete, then a workgroup barrier with no vmcnt wait.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// 16 consecutive activations of one row from global memory or LDS.
template <int XT>
__device__ __forceinline__ void load_frag(XRaw<XT>& f, const uint8_t* p) {
  if constexpr (XT == XT_S8) {
    f.v = *(const u32x4*)p;
  } else if constexpr (XT == XT_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f.v[i] = *(const f32x4*)(p + 16 * i);
  } else {
    typedef decltype(f.a) V;
    f.a = *(const V*)p;
    f.b = *(const V*)(p + 16);
  }
}

// s8 fragment (xq - 128) of 16 raw activations.
template <int XT>
__device__ __forceinline__ i32x4 quant16(const XRaw<XT>& f, float inv, float zpf) {
  uint32_t d[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    d[i] = pack_act_s8x4(__builtin_fmaf(f.get(4 * i), inv, zpf), __builtin_fmaf(f.get(4 * i + 1), inv, zpf),
                         __builtin_fmaf(f.get(4 * i + 2), inv, zpf), __builtin_fmaf(f.get(4 * i + 3), inv, zpf));
  return (i32x4){(int)d[0], (int)d[1], (int)d[2], (int)d[3]};
}

// LDS layout: [KS][G][64] partial tiles (16 bytes each), then per-wave
// (min, max) pairs, then the x copy.
template <int G>
__host__ __device__ constexpr int red_bytes(int ks) { return ks * G * 64 * 16; }
__host__ __device__ constexpr int mm_bytes() { return kFastMaxWaves * 8; }

__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}

// Fused greedy token (kGemvArgmax): `key` is this lane's best argmax_key over
// the outputs it stored.  The workgroup folds its keys per row (lanes, then
// its row tiles through `lds`, G * 16 keys) and merges them into the keys of
// its slot (slot = blockIdx.x % kArgmaxSlots) with an atomic max, then counts
// itself finished in its slot; the last workgroup of a slot counts the slot
// finished; the last slot gathers the keys of every slot (one per lane),
// writes each row's token and leaves the state at zero for the next launch.
// No workgroup waits for another.  Called by every wave.
//
// Every value that crosses workgroups travels through device-scope atomics,
// which the GPU performs at one point for all its XCDs, so no cache
// write-back or invalidation is needed (an agent-scope fence per workgroup
// costs an L2 write-back: measured 4.7x slower on the 151936-row lm_head).
// Atomics on one address are performed one after another, so the count and
// the keys are spread over slots (one count for all 4748 workgroups of the
// lm_head cost 14 us).  What matters is order: a workgroup's key updates
// are performed before its count, because the wave waits for their returned
// old values (vmcnt 0) before it issues the count, and each later step is
// issued only after the count it depends on has returned.
__device__ __forceinline__ void argmax_epilogue(uint8_t* state, int64_t* idx, unsigned long long key, int ks, int G,
                                                int M, unsigned long long* lds) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  key = umax64(key, __shfl_xor(key, 16, 64));
  key = umax64(key, __shfl_xor(key, 32, 64));
  if (ks < G && g == 0) lds[ks * 16 + r] = key;
  lds_barrier();
  if (ks != 0) return;
  const unsigned nblk = gridDim.x, slot = blockIdx.x % kArgmaxSlots;
  unsigned long long* const skeys = (unsigned long long*)(state + slot * kArgmaxSlotBytes);
  unsigned* const scount = (unsigned*)(state + slot * kArgmaxSlotBytes + 128);
  unsigned* const tcount = (unsigned*)(state + kArgmaxSlots * kArgmaxSlotBytes + 128);
  unsigned long long prior = 0;
  if (g == 0 && r < M) {
    unsigned long long best = 0;
    for (int j = 0; j < G; ++j) best = umax64(best, lds[j * 16 + r]);
    prior = __hip_atomic_fetch_max(skeys + r, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  asm volatile("" ::"v"(prior) : "memory");  // the returned old keys are in registers: the updates are performed
  wait_vm<0>();
  asm volatile("" ::: "memory");
  unsigned old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(scount, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __shfl(old, 0, 64);
  if (old != argmax_slot_members(nblk, slot, kArgmaxSlots) - 1) return;  // not the slot's last workgroup
  if (lane == 0) {
    __hip_atomic_store(scount, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __hip_atomic_fetch_add(tcount, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  old = __shfl(old, 0, 64);
  if (old != argmax_slots_used(nblk, kArgmaxSlots) - 1) return;  // not the last slot
  // every key is in place: lane l takes slot l's keys (clearing them), the
  // wave keeps each row's maximum
  unsigned long long k[16];
  const unsigned long long* lk = (const unsigned long long*)(state + lane * kArgmaxSlotBytes);
#pragma unroll
  for (int row = 0; row < 16; ++row)
    k[row] = row < M ? __hip_atomic_exchange((unsigned long long*)lk + row, 0ull, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT)
                     : 0ull;
#pragma unroll
  for (int row = 0; row < 16; ++row) {
    if (row < M) {  // uniform; a break here would keep the loop (and k[]) from unrolling
      unsigned long long v = k[row];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) v = umax64(v, __shfl_xor(v, o, 64));
      if (lane == 0) idx[row] = argmax_key_index(v);
    }
  }
  if (lane == 0) __hip_atomic_store(tcount, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

// QM: 0 weight-only; 1 W8A8 with the activation min/max partials of the
// pre-pass; 2 W8A8 that reduces min/max over the whole (small) x itself;
// 3 per-token symmetric W8A8 on pre-quantized s8 activations (XT_S8) with
// per-row scales a.rscale; 4 per-token symmetric W8A8 that reduces each row's
// max |x| and quantizes the rows itself.  QM 2 and 4 (and QM 1 with five row
// tiles) quantize x once per workgroup into s8 rows in LDS.
// GRP: grouped launch (a.nseg linears, see GemvArgs), weight-only or QM 2
// (each workgroup reduces the min/max of its own linear's x); a separate
// instance, so that the single-linear kernels carry no segment lookup.
template <int XT, int D, int G, bool XL, int QM, bool GRP = false>
__global__ __launch_bounds__(kFastMaxWaves * 64) void gemv_fast_kernel(GemvArgs a, int KW, int xch) {
  static_assert(!GRP || QM == 0 || QM == 2, "grouped launches: weight-only or fused int8-dyn");
  int bid = blockIdx.x;
  if constexpr (GRP) {
    {  // this workgroup's linear (uniform); fields read at constant indexes
       // only: a runtime index into the argument struct would move it to
       // private memory
#pragma unroll
      for (int i = 0; i < kGemvMaxSeg; ++i) {
        if (i < a.nseg && (int)blockIdx.x >= a.seg[i].wg0) {
          a.x = a.seg[i].x;
          a.packed = a.seg[i].packed;
          a.scale = a.seg[i].scale;
          a.bias = a.seg[i].bias;
          if constexpr (QM == 2) a.colsum = a.seg[i].colsum;
          a.y = a.seg[i].y;
          a.ldx = a.seg[i].ldx;
          a.ldy = a.seg[i].ldy;
          a.N = a.seg[i].N;
          a.Nt = a.seg[i].Nt;
          bid = (int)blockIdx.x - a.seg[i].wg0;
        }
      }
    }
  }
  constexpr bool W8A8 = QM != 0;
  constexpr bool PT = QM == 3;
  constexpr bool PTF = QM == 4;  // per-token, x quantized in the kernel
  static_assert(!PT || (XT == XT_S8 && !XL), "per-token: s8 fragments loaded directly");
  typedef typename std::conditional<W8A8, i32x4, f32x4>::type Acc;
  constexpr int EB = x_bytes<XT>();
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int KS = blockDim.x >> 6;
  const int tid = threadIdx.x, lane = tid & 63, ks = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int M = a.M, Kc = a.Kc, K = a.K;
  const int nt0 = bid * G;
  const int kbeg = ks * KW;
  const int cnt = min(KW, Kc - kbeg);  // >= 1: the host sizes KS so that every wave has a tile
  const int mr = min(r, M - 1);
  Acc* red = (Acc*)smem;
  float2* mmx = (float2*)(smem + red_bytes<G>(KS));
  uint8_t* xs = smem + red_bytes<G>(KS) + mm_bytes();
  const int xrow = K * EB;  // bytes of one x row in LDS
  constexpr bool kSplitX = XL && XT == XT_F32 && !W8A8;
  // five row tiles per workgroup (one workgroup per CU, up to 256 VGPRs per
  // wave): x goes to registers and only the planes take LDS
  constexpr bool kSplitReg = kSplitX && G == 5;
  // otherwise each wave copies and splits only its own K range of x (the
  // tiles it multiplies), in a region of its own: no workgroup barrier
  constexpr bool kSplitWave = kSplitX && !kSplitReg;
  const int sw_cap = (M * KW * 16 + 63) / 64 * 64;  // kSplitWave: 16-byte chunks per wave region
  uint8_t* xhi = xs + (kSplitReg ? 0 : KS * sw_cap * 16);  // kSplitX: bf16 planes [M][K] after the x copies
  uint8_t* xlo = xhi + M * K * 2;
  // kSplitX (M <= 8): MFMA column r < 8 multiplies the high plane of row r,
  // column r + 8 the remainder plane of the same row; the epilogue adds the
  // two columns
  const uint8_t* xpl = (r < 8 ? xhi : xlo) + min(r & 7, M - 1) * K * 2 + g * 16 * 2;
  // end of the x copy and planes: the fused argmax keeps G * 16 keys there
  // QM 2: x is quantized once, from the chunks each thread holds for the
  // min/max, into s8 rows [M][K] at xs (no x copy, no per-tile quantization)
  constexpr bool kQX = QM == 2;
  // QM 1 with five row tiles per workgroup: the (s_x, zp) of the pre-pass
  // partials quantize the thread's chunks of x, held in registers, the same way
  constexpr bool kQX1 = QM == 1 && G == 5;
  constexpr bool kQXL = kQX || kQX1 || PTF;  // s8 rows in LDS
  const int xend = kQXL ? M * K
                        : (kSplitX ? (kSplitReg ? 0 : KS * sw_cap * 16) + M * K * 4
                                   : (XL ? xch * (int)blockDim.x * 16 : 0));

  // epilogue operands of row tile `ks` (wave ks < G finishes tile ks)
  const int nte = min(nt0 + min(ks, G - 1), a.Nt - 1);
  const int ne = nte * 16 + 4 * g;
  f32x4 sc = {0.f, 0.f, 0.f, 0.f}, bi = {0.f, 0.f, 0.f, 0.f};
  i32x4 cs = {0, 0, 0, 0};
  if (ks < G) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int nn = min(ne + v, a.N - 1);
      sc[v] = a.scale[nn];
      if (a.bias) bi[v] = a.bias[nn];
      if constexpr (W8A8 && !PT && !PTF) cs[v] = a.colsum[nn];
    }
  }
  // W8A8: min/max partials of the activation pre-pass, or (QM 2) up to
  // FC 16-byte chunks of x per thread: chunk rounds past the end of x are
  // skipped (the condition is uniform over the workgroup), and the clamped
  // duplicates of a partial round are harmless
  constexpr int FC = G == 5 && XT == XT_F32 ? kFusedChunksWide : kFusedChunks;
  float2 part = {0.f, 0.f};
  u32x4 xmm[QM == 2 || PTF ? FC : 1];
  const int xm_nch = M * (K * EB / 16);  // QM 2: 16-byte chunks of x
  if constexpr (QM == 1) part = a.partials[min(tid, a.nparts - 1)];
  if constexpr (QM == 2 || PTF) {
    const int cpr = K * EB / 16;
#pragma unroll
    for (int i = 0; i < FC; ++i) {
      if (i * (int)blockDim.x >= xm_nch) {
        if constexpr (FC > kFusedChunks) continue;  // a break moves xmm to scratch
        else break;
      }
      const int c = min(tid + i * (int)blockDim.x, xm_nch - 1);
      const int m = c / cpr;
      xmm[i] = *(const u32x4*)((const uint8_t*)a.x + (int64_t)m * a.ldx * EB + (c - m * cpr) * 16);
    }
  }

  // x copy into LDS: xch 16-byte chunks per thread, sources clamped
  const uint8_t* xg = (const uint8_t*)a.x;
  u32x4 xq1[kQX1 ? kSplitRegChunks : 1];
  if constexpr (kQX1) {  // chunks c = tid + i * T of x, sources clamped
    const int cpr = K * EB / 16;
#pragma unroll
    for (int i = 0; i < kSplitRegChunks; ++i) {
      if (i * (int)blockDim.x < xm_nch) {
        const int c = min(tid + i * (int)blockDim.x, xm_nch - 1);
        const int m = c / cpr;
        xq1[i] = *(const u32x4*)(xg + (int64_t)m * a.ldx * EB + (c - m * cpr) * 16);
      }
    }
  }
  f32x4 xr[kSplitReg ? kSplitRegChunks : 1];
  if constexpr (kSplitReg) {  // chunks c = tid + i * T of x (row c / (K / 4)), sources clamped
    const int K4 = K / 4, xnch = M * K4;
#pragma unroll
    for (int i = 0; i < kSplitRegChunks; ++i) {
      if (i * (int)blockDim.x < xnch) {
        const int c = min(tid + i * (int)blockDim.x, xnch - 1);
        const int m = c / K4;
        xr[i] = *(const f32x4*)(xg + ((int64_t)m * a.ldx + (c - m * K4) * 4) * 4);
      }
    }
  } else if constexpr (kSplitWave) {
    // this wave's rows x[m][kbeg*64 .. (kbeg+cnt)*64): cnt * 16 chunks per row,
    // 64 per copy into consecutive slots of the wave's region, sources clamped
    const int cpw = cnt * 16, swn = M * cpw;
    uint8_t* xw = xs + ks * sw_cap * 16;
    for (int i = 0; i * 64 < swn; ++i) {
      const int j = min(i * 64 + lane, swn - 1);
      const int m = j / cpw;
      lds_copy16(xg + ((int64_t)m * a.ldx + (int64_t)kbeg * 64 + (j - m * cpw) * 4) * 4, xw + i * 64 * 16);
    }
  } else if constexpr (XL && !kQXL) {
    const int cpr = xrow / 16, nch = M * cpr;
    for (int i = 0; i < xch; ++i) {
      const int c0 = i * blockDim.x + ks * 64;  // first chunk of this wave
      const int c = min(c0 + lane, nch - 1);
      const int m = c / cpr;
      lds_copy16(xg + (int64_t)m * a.ldx * EB + (c - m * cpr) * 16, xs + c0 * 16);
    }
  }

  // first D tiles (and direct activations)
  const uint8_t* wp[G];
#pragma unroll
  for (int j = 0; j < G; ++j) wp[j] = a.packed + ((int64_t)min(nt0 + j, a.Nt - 1) * Kc + kbeg) * 1024 + lane * 16;
  const uint8_t* xp = xg + (int64_t)mr * a.ldx * EB + ((int64_t)kbeg * 64 + g * 16) * EB;
  u32x4 w[D][G];
  XRaw<XT> xd[XL || kQXL ? 1 : D];
#pragma unroll
  for (int p = 0; p < D; ++p) {
    const int kt = min(p, cnt - 1);
    if constexpr (!XL && !kQXL) load_frag<XT>(xd[p], xp + kt * 64 * EB);
#pragma unroll
    for (int j = 0; j < G; ++j) w[p][j] = load_tile_nt(wp[j] + kt * 1024);
  }

  // the 16 / EB activations of a 16-byte chunk of x as fp32
  constexpr int NE = 16 / EB;
  const auto chunk_vals = [](const u32x4& raw, float* v) {
#pragma unroll
    for (int j = 0; j < NE; ++j) {
      // copy the dword out first: a bit_cast of a vector-element lvalue
      // reads element 0 with this compiler
      const uint32_t word = raw[EB == 4 ? j : j / 2];
      if constexpr (XT == XT_F32) v[j] = __uint_as_float(word);
      else if constexpr (XT == XT_F16) v[j] = (float)__builtin_bit_cast(f16x2, word)[j & 1];
      else v[j] = (float)__builtin_bit_cast(bf16x2, word)[j & 1];
    }
  };
  ActQParams qp = {};
  float tok_s = 0.0f;  // PTF: the scale of row min(r, M - 1)
  if constexpr (XL || (W8A8 && !PT)) {
    if constexpr (QM == 2) {
      float mn = 0.0f, mx = 0.0f;
#pragma unroll
      for (int i = 0; i < FC; ++i) {
        if (i * (int)blockDim.x >= xm_nch) {
        if constexpr (FC > kFusedChunks) continue;  // a break moves xmm to scratch
        else break;
      }
        constexpr int NE = 16 / EB;
#pragma unroll
        for (int j = 0; j < NE; ++j) {
          // copy the dword out first: a bit_cast of a vector-element lvalue
          // reads element 0 with this compiler
          const uint32_t word = xmm[i][EB == 4 ? j : j / 2];
          float v;
          if constexpr (XT == XT_F32) v = __uint_as_float(word);
          else if constexpr (XT == XT_F16) v = (float)__builtin_bit_cast(f16x2, word)[j & 1];
          else v = (float)__builtin_bit_cast(bf16x2, word)[j & 1];
          mn = fminf(mn, v);
          mx = fmaxf(mx, v);
        }
      }
      part = make_float2(mn, mx);
    }
    if constexpr (W8A8 && !PTF) {
      const float mn = wave_min(part.x), mx = wave_max(part.y);
      if (lane == 0) mmx[ks] = make_float2(mn, mx);
    }
    if constexpr (PTF) {
      // per-row max |x| (the row quantizer's): per-wave maxima [KS][16] in
      // the partial-tile area, unused until the main loop ends
      float* rmx = (float*)smem;
      const int cpr = K * EB / 16;
      for (int m = 0; m < M; ++m) {
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < FC; ++i) {
          if (i * (int)blockDim.x >= xm_nch) {
        if constexpr (FC > kFusedChunks) continue;  // a break moves xmm to scratch
        else break;
      }
          const int c = min(tid + i * (int)blockDim.x, xm_nch - 1);
          if (c >= m * cpr && c < (m + 1) * cpr) {
            float v[NE];
            chunk_vals(xmm[i], v);
#pragma unroll
            for (int j = 0; j < NE; ++j) mx = fmaxf(mx, __builtin_fabsf(v[j]));
          }
        }
        mx = wave_max(mx);
        if (lane == 0) rmx[ks * 16 + m] = mx;
      }
    }
    if constexpr (XL) wait_vm<D * G>();  // this wave's x copies are in LDS; weights stay in flight
    if constexpr (!kSplitX) lds_barrier();  // (kSplitX: x from registers, or each wave's own copies)
    if constexpr (kSplitX) {
      // fp32 x: split once into bf16 high / remainder planes (hi + lo holds 16
      // significant bits of each activation, at fp32's exponent range).
      // Five-row-tile workgroups split the chunks their threads hold in
      // registers (c = tid + i * T), then wait at a workgroup barrier; the
      // other configurations split each wave's own K range (below).
      const int T = blockDim.x, xnch = M * (K / 4);
      const auto split_store = [&](const f32x4& v, int c) {
        bf16x4 h, l;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          __bf16 hh, ll;
          split_bf16(v[e], hh, ll);
          h[e] = hh;
          l[e] = ll;
        }
        *(bf16x4*)(xhi + c * 8) = h;  // element 4c of the [M][K] plane
        *(bf16x4*)(xlo + c * 8) = l;
      };
      if constexpr (kSplitReg) {
#pragma unroll
        for (int i = 0; i < kSplitRegChunks; ++i) {
          const int c = tid + i * T;
          if (i * T < xnch && c < xnch) split_store(xr[i], c);
        }
        lds_barrier();
      } else {
        // the lane's own copies (slot j = i * 64 + lane of the wave region),
        // four at a time; chunk j is row j / (cnt * 16), element
        // kbeg * 64 + 4 * (j % (cnt * 16)) of it
        const f32x4* rw = (const f32x4*)(xs + ks * sw_cap * 16);
        const int cpw = cnt * 16, swn = M * cpw;
        for (int b = 0; b * 64 < swn; b += 4) {
          f32x4 v[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] = rw[min((b + j) * 64 + lane, swn - 1)];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int jj = (b + j) * 64 + lane;
            if (jj < swn) {
              const int m = jj / cpw;
              split_store(v[j], (m * K + kbeg * 64) / 4 + (jj - m * cpw));
            }
          }
        }
        // the wave reads back only planes its own lanes wrote (its K range):
        // its LDS writes complete, no workgroup barrier
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        asm volatile("" ::: "memory");
      }
    }
    if constexpr (W8A8 && !PTF) {
      float mn = 0.0f, mx = 0.0f;
      for (int i = 0; i < KS; ++i) {
        const float2 v = mmx[i];
        mn = fminf(mn, v.x);
        mx = fmaxf(mx, v.y);
      }
      qp = choose_act_qparams(mn, mx);
    }
    if constexpr (PTF) {  // s = max(max |x|, 1e-8) / 127, the IEEE division of the row quantizer
      const float* rmx = (const float*)smem;
      const int rr = min(r, M - 1);
      float mx = rmx[rr];
      for (int i = 1; i < KS; ++i) mx = fmaxf(mx, rmx[i * 16 + rr]);
      tok_s = fmaxf(mx, 1e-8f) / 127.0f;
    }
    if constexpr (kQXL) {
      // the s8 values xq - 128 of this thread's chunks (quant16's arithmetic:
      // one fma and one pack per value), 16 / EB values per chunk; per-token:
      // clamp(rne(x / s), -127, 127), the row quantizer's values
      const int cpr = K * EB / 16;
      const auto quant_store = [&](const u32x4& raw, int c) {
        const int m = c / cpr;
        uint8_t* dst = xs + m * K + (c - m * cpr) * NE;
        float v[NE];
        chunk_vals(raw, v);
        uint32_t d[NE / 4];
        if constexpr (PTF) {
          const float sr = __shfl(tok_s, m, 64);  // lane m holds row m's scale
#pragma unroll
          for (int j = 0; j < NE / 4; ++j) {
            d[j] = 0u;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float q = __builtin_rintf(v[4 * j + e] / sr);
              q = fminf(fmaxf(q, -127.0f), 127.0f);
              d[j] |= ((uint32_t)(int)q & 0xffu) << (8 * e);
            }
          }
        } else {
#pragma unroll
          for (int j = 0; j < NE / 4; ++j)
            d[j] = pack_act_s8x4(__builtin_fmaf(v[4 * j], qp.inv, qp.zpf), __builtin_fmaf(v[4 * j + 1], qp.inv, qp.zpf),
                                 __builtin_fmaf(v[4 * j + 2], qp.inv, qp.zpf),
                                 __builtin_fmaf(v[4 * j + 3], qp.inv, qp.zpf));
        }
        if constexpr (NE == 4) *(uint32_t*)dst = d[0];
        else *(u32x2*)dst = (u32x2){d[0], d[1]};
      };
      if constexpr (kQX || PTF) {
#pragma unroll
        for (int i = 0; i < FC; ++i) {
          if (i * (int)blockDim.x >= xm_nch) {
        if constexpr (FC > kFusedChunks) continue;  // a break moves xmm to scratch
        else break;
      }
          quant_store(xmm[i], min(tid + i * (int)blockDim.x, xm_nch - 1));
        }
      } else {
#pragma unroll
        for (int i = 0; i < kSplitRegChunks; ++i)
          if (i * (int)blockDim.x < xm_nch) quant_store(xq1[i], min(tid + i * (int)blockDim.x, xm_nch - 1));
      }
      lds_barrier();
    }
  }

  Acc acc[G];
#pragma unroll
  for (int j = 0; j < G; ++j) acc[j] = Acc{0, 0, 0, 0};
  const uint8_t* xl = xs + mr * xrow + g * 16 * EB;
  auto step = [&](int p, int kt) {  // kt: tile index within this wave's range
    if constexpr (kSplitX) {
      const uint8_t* e = xpl + (kbeg + kt) * 64 * 2;
      const bf16x8 v0 = *(const bf16x8*)e, v1 = *(const bf16x8*)(e + 16);
#pragma unroll
      for (int j = 0; j < G; ++j) {
        bf16x8 w0, w1;
        u8x16_to_bf16(w[p][j], w0, w1);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0, v0, acc[j], 0, 0, 0);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1, v1, acc[j], 0, 0, 0);
      }
      return;
    }
    if constexpr (kQXL) {
      const i32x4 q = *(const i32x4*)(xs + mr * K + (kbeg + kt) * 64 + g * 16);
#pragma unroll
      for (int j = 0; j < G; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(tile_to_s8(w[p][j]), q, acc[j], 0, 0, 0);
      return;
    }
    XRaw<XT> f;
    if constexpr (XL) load_frag<XT>(f, xl + (kbeg + kt) * 64 * EB);
    else f = xd[p];
    if constexpr (PT) {
      const i32x4 q = __builtin_bit_cast(i32x4, f.v);
#pragma unroll
      for (int j = 0; j < G; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(tile_to_s8(w[p][j]), q, acc[j], 0, 0, 0);
    } else if constexpr (W8A8) {
      const i32x4 q = quant16<XT>(f, qp.inv, qp.zpf);
#pragma unroll
      for (int j = 0; j < G; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(tile_to_s8(w[p][j]), q, acc[j], 0, 0, 0);
    } else {
#pragma unroll
      for (int j = 0; j < G; ++j) tile_mma<XT>(w[p][j], f, acc[j]);
    }
  };
  int t = 0;
  for (; t + D < cnt; t += D) {
#pragma unroll
    for (int p = 0; p < D; ++p) {
      step(p, t + p);
      const int kt = min(t + D + p, cnt - 1);
      if constexpr (!XL && !kQXL) load_frag<XT>(xd[p], xp + kt * 64 * EB);
#pragma unroll
      for (int j = 0; j < G; ++j) w[p][j] = load_tile_nt(wp[j] + kt * 1024);
      // keep each refill next to the step that freed its registers (otherwise
      // the refills sink to the end of the batch and the ring drains)
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int p = 0; p < D; ++p)
    if (t + p < cnt) step(p, t + p);

  // cross-wave sum in wave order, epilogue by wave j for row tile j
  if (KS > 1) {
#pragma unroll
    for (int j = 0; j < G; ++j) red[(ks * G + j) * 64 + lane] = acc[j];
    lds_barrier();
  }
  // With a fused argmax every lane of every wave reaches the one call of
  // argmax_epilogue below with the wave reconverged: it holds a barrier and
  // cross-lane steps, so no lane may leave early or call it from a branch.
  const bool am = a.flags & kGemvArgmax;
  const int nt = nt0 + ks;
  const int n = nt * 16 + 4 * g;
  const auto tile_sum = [&]() {
    Acc s;
    if (KS > 1) {
      s = red[ks * 64 + lane];
      for (int i = 1; i < KS; ++i) s += red[(i * G + ks) * 64 + lane];
    } else {
      s = acc[0];  // one wave implies one row tile (the host keeps KS >= G)
    }
    return s;
  };
  Acc s{};
  if constexpr (kSplitX) {
    if (ks < G) {  // whole waves: column r + 8 (remainder plane) into column r
      s = tile_sum();
#pragma unroll
      for (int v = 0; v < 4; ++v) s[v] += __shfl_down(s[v], 8, 64);
    }
  }
  const bool live = ks < G && r < M && nt < a.Nt && n < a.N;
  if (!live && !am) return;
  unsigned long long key = 0;
  if (live) {
    if constexpr (!kSplitX) s = tile_sum();
    const int nvalid = min(4, a.N - n);
    f32x4 o;
    if constexpr (PT || PTF) {
      const float st = PT ? a.rscale[r] : tok_s;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if (a.acc_out && v < nvalid) a.acc_out[(int64_t)r * a.N + n + v] = s[v];
        const float mult = st * sc[v];
        o[v] = a.bias ? __builtin_fmaf((float)s[v], mult, bi[v]) : (float)s[v] * mult;
      }
    } else if constexpr (W8A8) {
      const int corr = 128 - qp.zp;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int av = s[v] + corr * cs[v];
        if (a.acc_out && v < nvalid) a.acc_out[(int64_t)r * a.N + n + v] = av;
        const float mult = qp.scale * sc[v];
        o[v] = a.bias ? __builtin_fmaf((float)av, mult, bi[v]) : (float)av * mult;
      }
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float out = s[v] * sc[v];
        if (a.bias) out = out + bi[v];
        o[v] = out;
      }
    }
    store_y4(a.y, a.yt, (int64_t)r * a.ldy + n, o, (a.flags & kGemvYVec) && nvalid == 4, nvalid);
    if (am) {  // fp32 y: the key of each stored value
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (v < nvalid) key = umax64(key, argmax_key(o[v], n + v));
    }
  }
  if (am) argmax_epilogue(a.am_state, a.idx, key, ks, G, M, (unsigned long long*)(xs + xend));
}

// Decode GEMV over MT 16-row tiles of x (16 < M <= 16 * MT, 64 | K, 16-byte
// aligned rows): weight-only on fp16 / bf16 activations, or int8-dyn (XT_S8)
// on the s8 rows xq - 128 of the quantize pre-pass with its (s_x, zp) and
// the GEMM's per-tensor epilogue.  The fast path's
// streaming of D weight tiles per step per wave, with MT activation fragments
// per tile (loaded directly from L2, D steps ahead like the weights).  Each
// weight tile is converted once and multiplied into MT accumulators; per-wave
// partials are summed through LDS in wave order, and wave j < G finishes
// weight tile j for every row tile.  The x bytes each workgroup reads grow
// with MT (all rows of x against its G weight tiles), so this pays up to
// M = 64; larger M runs the tiled GEMM.
template <int XT, int D, int G, int MT>
__global__ __launch_bounds__(kFastMaxWaves * 64) void gemv_mt_kernel(GemvArgs a, int KW) {
  static_assert(XT == XT_F16 || XT == XT_BF16 || XT == XT_S8, "fp16 / bf16 activations or s8 rows");
  constexpr bool I8 = XT == XT_S8;
  typedef typename std::conditional<XT == XT_F16, f16x8, bf16x8>::type V;
  typedef typename std::conditional<I8, i32x4, f32x4>::type Acc;
  constexpr int EB = I8 ? 1 : 2;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int KS = blockDim.x >> 6;
  const int tid = threadIdx.x, lane = tid & 63, ks = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int M = a.M, Kc = a.Kc;
  const int nt0 = blockIdx.x * G;
  const int kbeg = ks * KW;
  const int cnt = min(KW, Kc - kbeg);  // >= 1: the host sizes KS so that every wave has a tile
  Acc* red = (Acc*)smem;               // [KS][G][MT][64] partial tiles

  // epilogue operands of weight tile `ks` (wave ks < G finishes tile ks)
  const int nte = min(nt0 + min(ks, G - 1), a.Nt - 1);
  const int ne = nte * 16 + 4 * g;
  f32x4 sc = {0.f, 0.f, 0.f, 0.f}, bi = {0.f, 0.f, 0.f, 0.f};
  i32x4 cs = {0, 0, 0, 0};
  if (ks < G) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int nn = min(ne + v, a.N - 1);
      sc[v] = a.scale[nn];
      if (a.bias) bi[v] = a.bias[nn];
      if constexpr (I8) cs[v] = a.colsum[nn];
    }
  }

  // first D tiles and fragments (indexes clamped: no load is guarded)
  const uint8_t* wp[G];
#pragma unroll
  for (int j = 0; j < G; ++j) wp[j] = a.packed + ((int64_t)min(nt0 + j, a.Nt - 1) * Kc + kbeg) * 1024 + lane * 16;
  const uint8_t* xp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xp[mt] = (const uint8_t*)a.x + (int64_t)min(mt * 16 + r, M - 1) * a.ldx * EB + ((int64_t)kbeg * 64 + g * 16) * EB;
  u32x4 w[D][G];
  XRaw<XT> xd[D][MT];
#pragma unroll
  for (int p = 0; p < D; ++p) {
    const int kt = min(p, cnt - 1);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) load_frag<XT>(xd[p][mt], xp[mt] + kt * 64 * EB);
#pragma unroll
    for (int j = 0; j < G; ++j) w[p][j] = load_tile_nt(wp[j] + kt * 1024);
  }

  Acc acc[G][MT];
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[j][mt] = Acc{0, 0, 0, 0};
  auto step = [&](int p) {
#pragma unroll
    for (int j = 0; j < G; ++j) {
      if constexpr (I8) {
        const i32x4 wf = tile_to_s8(w[p][j]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[j][mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf, __builtin_bit_cast(i32x4, xd[p][mt].v), acc[j][mt], 0,
                                                             0, 0);
      } else {
        V w0, w1;
        if constexpr (XT == XT_F16)
          u8x16_to_f16(w[p][j], w0, w1);
        else
          u8x16_to_bf16(w[p][j], w0, w1);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if constexpr (XT == XT_F16) {
            acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w0, xd[p][mt].a, acc[j][mt], 0, 0, 0);
            acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w1, xd[p][mt].b, acc[j][mt], 0, 0, 0);
          } else {
            acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0, xd[p][mt].a, acc[j][mt], 0, 0, 0);
            acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1, xd[p][mt].b, acc[j][mt], 0, 0, 0);
          }
        }
      }
    }
  };
  int t = 0;
  for (; t + D < cnt; t += D) {
#pragma unroll
    for (int p = 0; p < D; ++p) {
      step(p);
      const int kt = min(t + D + p, cnt - 1);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) load_frag<XT>(xd[p][mt], xp[mt] + kt * 64 * EB);
#pragma unroll
      for (int j = 0; j < G; ++j) w[p][j] = load_tile_nt(wp[j] + kt * 1024);
      __builtin_amdgcn_sched_barrier(0);  // keep each refill next to the step that freed its registers
    }
  }
#pragma unroll
  for (int p = 0; p < D; ++p)
    if (t + p < cnt) step(p);

  // cross-wave sum in wave order; wave j < G finishes weight tile j
  if (KS > 1) {
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) red[((ks * G + j) * MT + mt) * 64 + lane] = acc[j][mt];
    lds_barrier();
  }
  const int nt = nt0 + ks;
  const int n = nt * 16 + 4 * g;
  if (ks >= G || nt >= a.Nt || n >= a.N) return;
  const int nvalid = min(4, a.N - n);
  const bool yvec = (a.flags & kGemvYVec) && nvalid == 4;
  float sx = 0.0f;
  int corr = 0;
  if constexpr (I8) {
    sx = a.qpbuf[0];
    corr = 128 - __float_as_int(a.qpbuf[1]);
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    Acc s;
    if (KS > 1) {
      s = red[(ks * MT + mt) * 64 + lane];
      for (int i = 1; i < KS; ++i) s += red[((i * G + ks) * MT + mt) * 64 + lane];
    } else {
      s = acc[0][mt];  // one wave implies one weight tile (the host keeps KS >= G)
    }
    const int m = mt * 16 + r;
    if (m >= M) continue;
    f32x4 o;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if constexpr (I8) {  // the per-tensor epilogue of the i8 GEMM
        const int av = s[v] + corr * cs[v];
        if (a.acc_out && v < nvalid) a.acc_out[(int64_t)m * a.N + n + v] = av;
        const float mult = sx * sc[v];
        o[v] = a.bias ? __builtin_fmaf((float)av, mult, bi[v]) : (float)av * mult;
      } else {
        float out = s[v] * sc[v];
        if (a.bias) out = out + bi[v];
        o[v] = out;
      }
    }
    store_y4(a.y, a.yt, (int64_t)m * a.ldy + n, o, yvec, nvalid);
  }
}

namespace {

// Instances: (D, G, XL).  XL uses LDS-resident x; direct modes keep D
// fragments in registers, so they use smaller D.
#define SBQ_FAST_CONFIGS(X) \
  X(0, 8, 1, true)          \
  X(1, 16, 1, true)         \
  X(2, 4, 1, false)         \
  X(3, 8, 1, false)         \
  X(4, 4, 2, false)         \
  X(5, 8, 2, false)         \
  X(6, 4, 2, true)          \
  X(7, 2, 5, true)          \
  X(8, 2, 6, false)

struct FastCfg {
  int id, D, G;
  bool XL;
};
constexpr FastCfg kFastCfgs[] = {
#define SBQ_FAST_ROW(id, D, G, XL) {id, D, G, XL},
    SBQ_FAST_CONFIGS(SBQ_FAST_ROW)
#undef SBQ_FAST_ROW
};
constexpr int kNumFastCfgs = sizeof(kFastCfgs) / sizeof(kFastCfgs[0]);

template <int XT, int QM, bool GRP = false>
int launch_fast_typed(int id, const GemvArgs& a, int ks, int KW, int xch, size_t lds, hipStream_t st) {
  const dim3 block(ks * 64);
  switch (id) {
#define SBQ_FAST_CASE(ID, D, G, XL)                                                                     \
  case ID:                                                                                              \
    if constexpr (QM != 3 || !XL) {                                                                     \
      hipLaunchKernelGGL((gemv_fast_kernel<XT, D, G, XL, QM, GRP>), dim3((a.Nt + G - 1) / G), block, lds, \
                         st, a, KW, xch);                                                               \
      return check_launch();                                                                            \
    }                                                                                                   \
    return -1;
    SBQ_FAST_CONFIGS(SBQ_FAST_CASE)
#undef SBQ_FAST_CASE
  }
  return -1;
}

}  // namespace

// Launch of fast-path configuration `id` with `ks` waves per workgroup
// (returns -1 when the configuration cannot run this shape).  W8A8 with
// a.nparts == 0 reduces the activation min/max in the kernel (x must fit
// kFusedChunks 16-byte chunks per thread of the workgroup, kFusedChunksWide for
// fp32 x with five row tiles).
int launch_gemv_fast_cfg(int id, int ks, const GemvArgs& a, int xt, bool w8a8, hipStream_t st) {
  if (id < 0 || id >= kNumFastCfgs || ks < 1 || ks > kFastMaxWaves) return -1;
  const FastCfg c = kFastCfgs[id];
  if (a.M < 1 || a.M > 16 || a.K != a.Kc * 64 || !(a.flags & 1)) return -1;
  const int KW = (a.Kc + ks - 1) / ks;
  ks = (a.Kc + KW - 1) / KW;  // every wave gets at least one K tile
  if (ks < c.G) return -1;                  // each row tile's epilogue belongs to one wave
  if (xt == XT_S8) {  // per-token W8A8 on pre-quantized activations: direct fragments only
    if (c.XL || !a.rscale) return -1;
    return launch_fast_typed<XT_S8, 3>(id, a, ks, KW, 0, (size_t)ks * c.G * 64 * 16 + mm_bytes(), st);
  }
  if (w8a8 && ks * 64 < a.nparts) return -1;  // one min/max partial per thread
  const int eb = xt == XT_F32 ? 4 : 2;
  const int64_t xbytes = (int64_t)a.M * a.K * eb;
  const bool split = c.XL && xt == XT_F32 && !w8a8;  // fp32 x: raw copy + fp16 planes
  const bool split_reg = split && c.G == 5;  // fp32 x in registers, planes only in LDS
  const bool qx1 = w8a8 && a.nparts > 0 && c.G == 5;  // pre-pass (s_x, zp), x quantized from registers
  if (c.XL && xbytes > (split_reg || qx1 ? kSplitWideBytes
                                         : (split ? kFastSplitBytes : (c.G == 5 ? kFastXLdsWideBytes : kFastXLdsBytes))))
    return -1;
  if (split && a.M > 8) return -1;  // the two planes of a row share the 16 MFMA columns
  if (c.D * c.G > 32) return -1;
  const int T = ks * 64;
  // per-token W8A8 with x quantized in the kernel: QM 4
  const int qm = !w8a8 ? 0 : ((a.flags & kGemvPerToken) ? 4 : (a.nparts > 0 ? 1 : 2));
  if (qm == 4 && (a.M > 16 || a.nparts > 0)) return -1;
  const int xch = c.XL && qm != 2 && qm != 4 && !split_reg && !qx1 ? (int)((xbytes / 16 + T - 1) / T) : 0;
  if ((split_reg || qx1) && (xbytes / 16 + T - 1) / T > kSplitRegChunks) return -1;  // the chunks each thread holds
  if (split && xch > kSplitChunks) return -1;  // the chunks of x each thread splits
  size_t lds = (size_t)ks * c.G * 64 * 16 + mm_bytes() + (c.XL && !split ? (size_t)xch * T * 16 : 0);
  if (split && !split_reg) lds += (size_t)ks * ((a.M * KW * 16 + 63) / 64 * 64) * 16;  // each wave's x copy
  if (split) lds += (size_t)xbytes;               // bf16 high / remainder planes
  if (qm == 2 || qm == 4 || qx1) lds += (size_t)a.M * a.K;  // the quantized s8 rows
  if (a.flags & kGemvArgmax) lds += (size_t)c.G * 16 * 8;  // the fused argmax's keys per row tile
  if ((qm == 2 || qm == 4) && xbytes > (int64_t)(c.G == 5 && xt == XT_F32 ? kFusedChunksWide : kFusedChunks) * 16 * T)
    return -1;  // every thread holds its chunks of x
#define SBQ_FAST_QM(XT_)                                                  \
  switch (qm) {                                                           \
    case 0:                                                               \
      return a.nseg > 1 ? launch_fast_typed<XT_, 0, true>(id, a, ks, KW, xch, lds, st) \
                        : launch_fast_typed<XT_, 0>(id, a, ks, KW, xch, lds, st);      \
    case 1: return launch_fast_typed<XT_, 1>(id, a, ks, KW, xch, lds, st); \
    case 2:                                                               \
      return a.nseg > 1 ? launch_fast_typed<XT_, 2, true>(id, a, ks, KW, xch, lds, st) \
                        : launch_fast_typed<XT_, 2>(id, a, ks, KW, xch, lds, st);      \
    default: return launch_fast_typed<XT_, 4>(id, a, ks, KW, xch, lds, st); \
  }
  switch (xt) {
    case XT_F16: SBQ_FAST_QM(XT_F16)
    case XT_BF16: SBQ_FAST_QM(XT_BF16)
    case XT_F32: SBQ_FAST_QM(XT_F32)
  }
#undef SBQ_FAST_QM
  return -2;
}

// Grouped launch of configuration `id`: a.seg[0 .. a.nseg) hold the linears
// (x, weights, scales, bias, column sums, y, strides, N, Nt); every linear
// gets ceil(Nt / G) workgroups of the grid, in segment order.  M, K, the
// dtypes and the flags are shared.  w8a8: int8-dyn with the min/max of each
// linear's x reduced in the kernel (QM 2; x within its fused capacity).
// Returns -1 when the configuration cannot run the shape.
int launch_gemv_fast_grouped(int id, int ks, GemvArgs a, int xt, bool w8a8, hipStream_t st) {
  if (id < 0 || id >= kNumFastCfgs || a.nseg < 2 || a.nseg > kGemvMaxSeg) return -1;
  const int G = kFastCfgs[id].G;
  int64_t wg = 0;
  for (int s = 0; s < a.nseg; ++s) {
    a.seg[s].wg0 = (int)wg;
    wg += (a.seg[s].Nt + G - 1) / G;
  }
  if (wg * G > 0x7fffffff / 16) return -1;
  // the launch-wide fields describe the whole grid (the kernel takes each
  // workgroup's operands from its segment)
  a.Nt = (int)(wg * G);
  a.N = a.Nt * 16;
  a.x = a.seg[0].x;
  a.ldx = a.seg[0].ldx;
  a.nparts = 0;
  a.flags &= ~(kGemvArgmax | kGemvPerToken);
  return launch_gemv_fast_cfg(id, ks, a, xt, w8a8, st);
}

// Decode over several 16-row tiles of x (gemv_mt_kernel): weight-only on fp16
// / bf16 x, or int8-dyn on the s8 rows of the quantize pre-pass (xt XT_S8,
// a.qpbuf and a.colsum set); aligned rows, 16 < M <= 64, 64 | K.  -1: not
// this path.  Every workgroup reads all of x, and the launch time grows with
// the x bytes its grid reads from L2 (MI355X: about 0.13-0.16 us per MB
// beyond a 2-5 us base).  gemm_alt: the tiled GEMM's mid-sized-M plan (64 x 64
// blocks, K split when the grid is small) is available to the caller; it is
// faster except on narrow layers with little x to read (measured, the GEMM
// alone against this kernel: int8-dyn N = 4096, K = 4096, M = 24 / 32 / 48:
// 7.8 / 8.6 / 10.7 us here against 9.9 / 9.8 / 10.0; N = 9728, K = 2560,
// M = 32: 13.9 against 10.8; weight-only, whose GEMM also needs its row-sum
// pre-pass, N = 4096, M = 24 / 32: 9.6 / 11.1 against 11.7 us plus the
// pre-pass), so with it the path is kept for N <= 4096 while the grid's x
// reads stay within 36 MB (s8) / 80 MB (fp16, bf16).  Without it, up to
// 90 MB / 120 MB, where this kernel beats the general GEMV and the unsplit
// GEMM (N = 4096, M = 24 / 33 / 48: 10.4 / 20.1 / 20.1 -> 9.4 / 12.0 / 15.1 us).
bool gemv_mt_applies(int64_t M, int64_t K, int64_t N, int xt, bool gemm_alt) {
  if (!(xt == XT_F16 || xt == XT_BF16 || xt == XT_S8) || M <= 16 || M > 64 || K % 64 != 0) return false;
  const int64_t Nt = (N + 15) / 16, Kc = K / 64;
  const int G = Kc < 128 && Nt >= 384 ? 2 : 1;
  const int64_t x_grid_bytes = M * K * (xt == XT_S8 ? 1 : 2) * ((Nt + G - 1) / G);
  if (gemm_alt) return Nt <= 256 && x_grid_bytes <= ((int64_t)(xt == XT_S8 ? 36 : 80) << 20);
  return x_grid_bytes <= ((int64_t)(xt == XT_S8 ? 90 : 120) << 20);
}

int launch_gemv_mt(const GemvArgs& a, int xt, hipStream_t st, bool gemm_alt) {
  if (a.K != a.Kc * 64 || !(a.flags & kGemvXVec) || !gemv_mt_applies(a.M, a.K, a.N, xt, gemm_alt)) return -1;
  if (xt == XT_S8 && (!a.qpbuf || !a.colsum)) return -1;
  const int mt = (a.M + 15) / 16;
  const bool wide = a.Kc < 128 && a.Nt >= 384;
  const int G = wide ? 2 : 1;
  int ks = 4;
  const int KW = (a.Kc + ks - 1) / ks;
  ks = (a.Kc + KW - 1) / KW;  // every wave gets at least one K tile
  if (ks < G) return -1;
  const size_t lds = (size_t)ks * G * mt * 64 * 16;
  const dim3 grid((unsigned)((a.Nt + G - 1) / G)), block(ks * 64);
#define SBQ_MT_CASE(XT_, G_, MT_)                                                                \
  if (xt == XT_ && G == G_ && mt == MT_) {                                                      \
    hipLaunchKernelGGL((gemv_mt_kernel<XT_, 4, G_, MT_>), grid, block, lds, st, a, KW);         \
    return check_launch();                                                                      \
  }
  SBQ_MT_CASE(XT_F16, 1, 2) SBQ_MT_CASE(XT_F16, 1, 3) SBQ_MT_CASE(XT_F16, 1, 4)
  SBQ_MT_CASE(XT_F16, 2, 2) SBQ_MT_CASE(XT_F16, 2, 3) SBQ_MT_CASE(XT_F16, 2, 4)
  SBQ_MT_CASE(XT_BF16, 1, 2) SBQ_MT_CASE(XT_BF16, 1, 3) SBQ_MT_CASE(XT_BF16, 1, 4)
  SBQ_MT_CASE(XT_BF16, 2, 2) SBQ_MT_CASE(XT_BF16, 2, 3) SBQ_MT_CASE(XT_BF16, 2, 4)
  SBQ_MT_CASE(XT_S8, 1, 2) SBQ_MT_CASE(XT_S8, 1, 3) SBQ_MT_CASE(XT_S8, 1, 4)
  SBQ_MT_CASE(XT_S8, 2, 2) SBQ_MT_CASE(XT_S8, 2, 3) SBQ_MT_CASE(XT_S8, 2, 4)
#undef SBQ_MT_CASE
  return -1;
}

// Fast-path choice for a shape (false: the general kernel runs).  Measured on
// MI355X over the decode shapes (M = 1, 4, 16; K = 4096, 12288; N = 4096 ..
// 151936): 4-tile steps over two row tiles per wave for wide K = 4096 layers,
// 8-tile steps over one row tile for long K or narrow N, two waves per row tile
// once M > 8 (the activation fragments then dominate the registers), five row
// tiles per workgroup with x in LDS at M = 4 .. 8 on wide short-K layers, six
// with x loaded directly where five do not fit one round at M > 8.  bf16
// activations follow the fp16 rules; fp32 activations are copied to LDS and
// split once into bf16 high / remainder planes when x fits (M <= 8), and
// otherwise take direct steps with two row tiles per wave on wide layers (M =
// 4, N = 6144 and 24576: 21-28% faster than one row tile).
bool pick_gemv_fast(int64_t M, int64_t K, int64_t N, int xt, bool w8a8, bool xvec, int* id, int* ks) {
  if (M < 1 || M > 16 || K % 64 != 0 || !xvec) return false;
  const int64_t Kc = K / 64, Nt = (N + 15) / 16;
  if (xt == XT_F32) {
    // x in LDS (weight-only, M <= 8: split once into bf16 planes) when it
    // fits 24 KiB, or 48 KiB for one row (M = 1, K = 12288: 16% faster than
    // direct steps; the raw copy and the planes then hold 96 KiB of LDS, one
    // workgroup per CU).  One row of a wide layer takes 4-tile steps over two
    // row tiles per wave with 8 waves per workgroup (half the copies and
    // splits: QKV and gate+up at K = 4096 2-6% faster) unless that grid needs
    // fewer rounds of the 256 CUs than one row tile per workgroup
    // (measured on MI355X at M = 1: N = 19456 and 18820 at K = 2560, 14.0 ->
    // 12.0 us; N = 5120, K = 4096 keeps two tiles, 7.9 -> 7.2 us against one).
    // Long K over at most 256 row tiles takes 8 waves (N = 2560, K = 9728:
    // 8.9 -> 8.5 us; N = 4096, K = 12288: 11.6 -> 11.35 us).  Else direct steps: 8 tiles over one row tile for long
    // K, 4 tiles over two row tiles for wide layers, 4 tiles over one row
    // tile otherwise; K <= 256 one wave of 4-tile steps (K = 128: 3.0 ->
    // 2.65 us).
    const int64_t xb = M * K * 4;
    const bool xl = (w8a8 || M <= 8) && (xb <= 24576 || (!w8a8 && M == 1 && xb <= kFastSplitBytes));
    const auto rounds = [](int64_t wgs) { return (wgs + 255) / 256; };
    const bool wide1 = xl && !w8a8 && M == 1 && Kc < 128 && Nt > 256 && rounds(Nt) >= 2 * rounds((Nt + 1) / 2);
    *id = wide1 ? 6 : (xl ? 0 : (Kc >= 128 ? 3 : (Nt >= 384 ? 4 : 2)));
    *ks = wide1 || (xl && !w8a8 && Kc >= 128 && Nt <= 256) ? 8 : 4;
    if (!w8a8 && Kc <= 4) {
      *id = 2;
      *ks = 1;
    }
    // M = 4 .. 8 on a wide short-K layer whose grid of five row tiles per
    // workgroup fits one round of the CUs: x (up to 80 KiB) loaded into
    // registers and split into planes in LDS, read once per five row tiles
    if (!w8a8 && M >= 4 && M <= 8 && Kc < 128 && Nt > 1024 && (Nt + 4) / 5 <= 256 && xb <= kSplitWideBytes) {
      *id = 7;  // D=2, G=5, x in LDS
      *ks = 8;
    }
  } else if (M <= 8) {
    // two row tiles per workgroup for wide layers; weight-only also from 257
    // row tiles, where one tile per workgroup needs a second round of the 256
    // CUs (M = 1, N = 5120, K = 4096: 7.06 -> 5.87 us), and so does W8A8 on
    // more than 32 KiB of x, which every workgroup of the fused min/max reads
    // whole: half the workgroups halve those reads
    const bool wide = Kc < 128 && (Nt >= 384 || (Nt > 256 && (!w8a8 || M * K * 2 > 32768)));
    *id = wide ? 4 : 3;  // D=4, G=2 | D=8, G=1
    *ks = 4;
    if (!w8a8) {
      // Measured on MI355X at M = 1, 4, 8 (fp16 x, interleaved timings of
      // every configuration):
      // * K <= 256: one wave of 4-tile steps (lora_*[1], K = 128: 2.65 ->
      //   2.39 us at M = 1, 2.92 -> 2.46 at M = 8);
      // * x in LDS, one row tile per workgroup, when x fits: on layers of
      //   fewer than 256 row tiles (N = 4 .. 3000: 0.1-0.4 us per launch), and
      //   on wide layers whose two-tile grid takes more rounds of 256 CUs
      //   than the one-tile grid (N = 18820: 15.0 -> 14.2 us, N = 10000:
      //   10.2 -> 9.2 us; N = 6144, 8192, 24576 and 151936 keep two tiles).
      const auto rounds = [](int64_t wgs) { return (wgs + 255) / 256; };
      const bool xl = M * K * 2 <= kFastXLdsBytes;
      if (Kc <= 4) {
        *id = 2;  // D=4, G=1
        *ks = 1;
      } else if (xl && (wide ? rounds(Nt) < 2 * rounds((Nt + 1) / 2) : Nt < 256)) {
        *id = 0;  // D=8, G=1, x in LDS
      }
      // M = 4 .. 8, a wide layer at short K whose grid of five row tiles per
      // workgroup fills one round of the CUs: x (up to 64 KiB) in LDS, read
      // once per five row tiles instead of once per one or two (M = 8, N =
      // 19456 / 18820, K = 2560: 12.5 -> 10.9 / 12.7 -> 10.7 us; M = 4: 11.9
      // -> 10.5 / 11.8 -> 10.3 us; grids of more than 256 such workgroups, as
      // N = 24576 at K = 4096, run slower)
      if (M >= 4 && Kc < 128 && Nt > 1024 && (Nt + 4) / 5 <= 256 && M * K * 2 <= kFastXLdsWideBytes) {
        *id = 7;  // D=2, G=5, x in LDS
        *ks = 8;
      }
    }
  } else {
    const bool wide = Kc <= 64 && Nt >= 384;
    *id = wide ? 5 : 3;  // D=8, G=2 | D=8, G=1
    *ks = 2;
    // five row tiles per workgroup with x in LDS, as at M = 4 .. 8
    if (!w8a8 && Kc < 128 && Nt > 1024 && (Nt + 4) / 5 <= 256 && M * K * 2 <= kFastXLdsWideBytes) {
      *id = 7;  // D=2, G=5, x in LDS
      *ks = 8;
    } else if (!w8a8 && Kc < 128 && Nt > 1024 && (Nt + 5) / 6 <= 256) {
      // six row tiles per workgroup, x fragments loaded directly: each wave
      // reads its K range of x once per six row tiles instead of two, and the
      // grid still fits one round of the CUs (M = 16, N = 24576, K = 4096:
      // 19.8 -> 18.2 us; M = 16 x is 128 KiB there, beyond the LDS copy)
      *id = 8;  // D=2, G=6
      *ks = 8;
    }
  }
  if (w8a8) {
    // the activation min/max is reduced in the kernel for x <= 64 KiB (up to
    // 8 chunks of 16 bytes per thread, one pre-pass launch less: M = 1..4
    // decode 8-24% faster); 8 waves beyond 32 KiB and on the widest layers
    const int64_t xb = M * K * (xt == XT_F32 ? 4 : 2);
    if (xb > 16384 && xb <= 65536 && (xb > 32768 || Nt >= 1024)) *ks = 8;
    if (Kc <= 4 && xb <= (int64_t)kFusedChunks * 16 * 64) {  // short K: one wave, as for weight-only
      *id = 2;
      *ks = 1;
    } else if (*ks < kFusedMinWaves) {
      *ks = kFusedMinWaves;  // 256 threads cover the min/max partials / fused x
    }
    // M = 4 .. 8 on a wide short-K layer: five row tiles per workgroup, as
    // for weight-only: x up to 64 KiB with the fused min/max (8 chunks per
    // thread; fp32 x up to 80 KiB, 10 chunks, so that M = 8 at K = 2560
    // takes no pre-pass launch: checkpoint int8-dyn step 3036 -> 3240 tok/s),
    // up to 80 KiB after the min/max pre-pass
    if (M >= 4 && Kc < 128 && Nt > 1024 && (Nt + 4) / 5 <= 256 && xb <= kSplitWideBytes) {
      *id = 7;
      *ks = 8;
    }
  }
  return true;
}

}  // namespace sbq

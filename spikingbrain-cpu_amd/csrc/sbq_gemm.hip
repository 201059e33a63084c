// sbq_gemm.hip - prefill (large-M) quantized linear, MFMA bound.
//
// Replaces spikingbrain_cpu/quant.py:41-53 (Int8Linear.forward) and
// quant.py:63-66 (DynamicInt8Linear.forward) for the prompt chunks the model
// feeds (model.py:439: up to 512 tokens per chunk) and larger batches.
//
// Block tile BN (output channels) x BM (tokens) x 64*KT (K per stage; KT = 2
// on most W8A8 configurations), WN x WM waves.  Each stage copies BN/16 packed
// weight tiles per K tile verbatim into LDS and the BM x 64 activation slab
// into an XOR-swizzled LDS tile, straight from global memory (LDS DMA); later
// stages land while MFMAs run on the current one (one barrier per stage).
//   W-only: fp16 activations meet the weights as fp16 subnormals
//           (q + 128) * 2^-24 (one v_perm per pair) and the epilogue removes
//           128 * rowsum(x); bf16 activations meet exact bf16 weights.  Both
//           run v_mfma_f32_16x16x32_{f16,bf16}.  With a workspace, fp32 and
//           bf16 activations are first staged as a row-scaled fp16 plane (fp32:
//           11 significant bits) for the fp16 kernel; without one, fp32 runs as bf16
//           hi + lo planes in the register-staged kernel.  Epilogue:
//           * scale[n] (+ bias[n]).
//   W8A8:   the activations are quantized to s8 (xq - 128) once, by a
//           pre-pass into the workspace; weights are used as s8,
//           v_mfma_i32_16x16x64_i8 accumulates exactly; the epilogue adds
//           (128 - zp) * colsum[n] and applies fp32(s_x * scale[n]) (+ bias[n]
//           fused), as fbgemm does.
#include <type_traits>

#include "sbq_common.h"
#include "sbq_dma.h"
#include "sbq_gemv_ops.h"
#include "sbq_index.h"
#include "sbq_launch.h"

namespace sbq {

// LDS activation tile for 2-byte operands: 64 K-columns per row = 8 chunks of
// 16 bytes; chunk c of row r lives at slot c ^ (r & 7) so that the 16 rows a
// quarter-wave reads for one fragment spread over all banks.
__device__ __forceinline__ int xs_off(int row, int chunk) { return row * 128 + ((chunk ^ (row & 7)) << 4); }

template <int XT>
struct GemmOp;
template <>
struct GemmOp<XT_F16> {
  typedef f16x8 V;
  static constexpr int NS = 1;
  static __device__ __forceinline__ void wconv(u32x4 w, V& a, V& b) { u8x16_to_f16(w, a, b); }
  static __device__ __forceinline__ f32x4 mma(V a, V b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct GemmOp<XT_BF16> {
  typedef bf16x8 V;
  static constexpr int NS = 1;
  static __device__ __forceinline__ void wconv(u32x4 w, V& a, V& b) { u8x16_to_bf16(w, a, b); }
  static __device__ __forceinline__ f32x4 mma(V a, V b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct GemmOp<XT_F32> {
  typedef bf16x8 V;
  static constexpr int NS = 2;
  static __device__ __forceinline__ void wconv(u32x4 w, V& a, V& b) { u8x16_to_bf16(w, a, b); }
  static __device__ __forceinline__ f32x4 mma(V a, V b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

// Convert 8 fp32 activations into the operand plane(s) (16 bytes each).
template <int XT>
__device__ __forceinline__ void x8_to_planes(const float* t, u32x4* planes) {
  if constexpr (XT == XT_F16) {
    f16x8 h;
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = (_Float16)t[j];
    planes[0] = __builtin_bit_cast(u32x4, h);
  } else if constexpr (XT == XT_BF16) {
    bf16x8 h;
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = (__bf16)t[j];
    planes[0] = __builtin_bit_cast(u32x4, h);
  } else {
    bf16x8 h, l;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      __bf16 a, b;
      split_bf16(t[j], a, b);
      h[j] = a;
      l[j] = b;
    }
    planes[0] = __builtin_bit_cast(u32x4, h);
    planes[1] = __builtin_bit_cast(u32x4, l);
  }
}

// Raw 16-byte chunk load for 2-byte activations on the fast path (no
// conversion through fp32).
template <int XT>
__device__ __forceinline__ void load_x_chunk(const void* x, int64_t ldx, int M, int K, int m, int k0, bool xvec,
                                             u32x4* planes) {
  if constexpr (XT != XT_F32) {
    if (m < M && xvec && k0 + 8 <= K) {
      planes[0] = *(const u32x4*)((const uint16_t*)x + (int64_t)m * ldx + k0);
      return;
    }
  }
  float t[8];
  load8_f32<XT>(x, ldx, M, K, m, k0, xvec, t);
  x8_to_planes<XT>(t, planes);
}

template <int XT, int BN, int BM, int WN, int WM>
__global__ __launch_bounds__(WN* WM * 64) void gemm_w8_kernel(const void* __restrict__ x, int64_t ldx, int M,
                                                              int K, int Kc, const uint8_t* __restrict__ packed,
                                                              const float* __restrict__ scale,
                                                              const float* __restrict__ bias, int N, int Nt,
                                                              void* __restrict__ y, int yt, int64_t ldy,
                                                              int flags) {
  typedef GemmOp<XT> Op;
  typedef typename Op::V V;
  constexpr int NS = Op::NS;
  constexpr int NT = WN * WM * 64;
  constexpr int TN = BN / WN, TM = BM / WM;
  constexpr int FN = TN / 16, FM = TM / 16;
  constexpr int WCH = BN * 4 / NT;  // 16-byte weight chunks per thread per stage
  constexpr int XCH = BM * 8 / NT;  // 16-byte activation chunks (8 values) per thread per stage
  static_assert(WCH * NT == BN * 4 && XCH * NT == BM * 8, "tile/thread mismatch");

  __shared__ __attribute__((aligned(16))) uint8_t wl[2][BN * 64];
  __shared__ __attribute__((aligned(16))) uint8_t xl[2][NS][BM * 128];

  const bool xvec = flags & 1, yvec = flags & 2;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int r = lane & 15, g = lane >> 4;
  const int wn = wave / WM, wm = wave % WM;
  const int nt0 = blockIdx.x * (BN / 16);
  const int m0 = blockIdx.y * BM;

  u32x4 wreg[WCH];
  u32x4 xreg[XCH][NS];

  auto gload = [&](int kc) {
#pragma unroll
    for (int i = 0; i < WCH; ++i) {
      const int c = tid + i * NT;
      const int j = c >> 6, slot = c & 63;
      if (nt0 + j < Nt) wreg[i] = *(const u32x4*)(packed + ((int64_t)(nt0 + j) * Kc + kc) * 1024 + slot * 16);
    }
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int c = tid + i * NT;
      const int row = c >> 3, ch = c & 7;
      load_x_chunk<XT>(x, ldx, M, K, m0 + row, kc * 64 + ch * 8, xvec, xreg[i]);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < WCH; ++i) {
      const int c = tid + i * NT;
      *(u32x4*)(&wl[buf][c * 16]) = wreg[i];
    }
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int c = tid + i * NT;
      const int row = c >> 3, ch = c & 7;
#pragma unroll
      for (int h = 0; h < NS; ++h) *(u32x4*)(&xl[buf][h][xs_off(row, ch)]) = xreg[i][h];
    }
  };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int a = 0; a < FN; ++a)
#pragma unroll
    for (int b = 0; b < FM; ++b) acc[a][b] = (f32x4){0.f, 0.f, 0.f, 0.f};

  gload(0);
  sstore(0);
  __syncthreads();

  for (int kc = 0; kc < Kc; ++kc) {
    const int buf = kc & 1;
    if (kc + 1 < Kc) gload(kc + 1);

    V wf[FN][2];
#pragma unroll
    for (int a = 0; a < FN; ++a) {
      const u32x4 w = *(const u32x4*)(&wl[buf][(wn * FN + a) * 1024 + lane * 16]);
      Op::wconv(w, wf[a][0], wf[a][1]);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int b = 0; b < FM; ++b) {
        const int row = wm * TM + b * 16 + r;
        V xf[NS];
#pragma unroll
        for (int h = 0; h < NS; ++h) xf[h] = *(const V*)(&xl[buf][h][xs_off(row, 2 * g + s)]);
#pragma unroll
        for (int a = 0; a < FN; ++a) {
#pragma unroll
          for (int h = NS - 1; h >= 0; --h) acc[a][b] = Op::mma(wf[a][s], xf[h], acc[a][b]);
        }
      }
    }
    if (kc + 1 < Kc) sstore(buf ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds y[m0 + wm*TM + b*16 + r][n0 + (wn*FN + a)*16 + 4g + v]
#pragma unroll
  for (int a = 0; a < FN; ++a) {
    const int n = (nt0 + wn * FN + a) * 16 + 4 * g;
    if (n >= N) continue;
    const int nvalid = min(4, N - n);
    f32x4 sc, bi;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int nn = min(n + v, N - 1);
      sc[v] = scale[nn];
      bi[v] = bias ? bias[nn] : 0.0f;
    }
#pragma unroll
    for (int b = 0; b < FM; ++b) {
      const int m = m0 + wm * TM + b * 16 + r;
      if (m >= M) continue;
      f32x4 o;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float out = acc[a][b][v] * sc[v];
        if (bias) out = out + bi[v];
        o[v] = out;
      }
      store_y4(y, yt, (int64_t)m * ldy + n, o, yvec && nvalid == 4, nvalid);
    }
  }
}

// ---------------------------------------------------------------------------
// Direct-to-LDS pipelined GEMM (weight-only, fp16/bf16 activations, K % 64 == 0)
//
// Block tile BN output channels x BM tokens x 64 K, WN x WM waves.  Used with
// 256 x 128, 8 waves (4 x 2, wave tile 64 x 64) and 2 stages: measured on
// MI355X this beats 4-wave / 3-stage variants, because two 64 KiB workgroups
// share a CU (4 waves per SIMD) and hide each other's LDS and barrier stalls.
// Each stage is filled by buffer_load_dwordx4 ... lds (16 bytes per lane
// straight into LDS, no register staging): the packed weight tiles land
// verbatim, the activation rows land with their 16-byte chunks XOR-swizzled by
// ((row >> 1) & 7), which spreads the 16 rows one ds_read_b128 quarter-wave
// touches over all 64 LDS banks.  With NS stages, NS-1 are in flight while one
// is multiplied.
// Rows >= M and tiles >= Nt are loaded from clamped (in-bounds) addresses and
// never stored.
// ---------------------------------------------------------------------------



// Most workgroups K is split over (the split-K plan's largest split).
constexpr int kMaxSplits = 4;


// Wait until only the `younger` most recent stages (LPS DMA instructions each)
// of this wave are still in flight.
template <int LPS, int NS>
__device__ __forceinline__ void wait_stages(int younger) {
  static_assert(LPS * (NS - 2) < 64, "vmcnt range");
  if constexpr (NS > 7) { if (younger >= 6) { wait_vmcnt<(NS > 7 ? 6 * LPS : 0)>(); return; } }
  if constexpr (NS > 6) { if (younger == 5) { wait_vmcnt<(NS > 6 ? 5 * LPS : 0)>(); return; } }
  if constexpr (NS > 5) { if (younger == 4) { wait_vmcnt<(NS > 5 ? 4 * LPS : 0)>(); return; } }
  if constexpr (NS > 4) { if (younger == 3) { wait_vmcnt<(NS > 4 ? 3 * LPS : 0)>(); return; } }
  if constexpr (NS > 3) { if (younger == 2) { wait_vmcnt<(NS > 3 ? 2 * LPS : 0)>(); return; } }
  if constexpr (NS > 2) { if (younger == 1) { wait_vmcnt<(NS > 2 ? LPS : 0)>(); return; } }
  wait_vmcnt<0>();
}


__device__ __forceinline__ int xsw_off(int row, int chunk) { return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4); }

// Arguments of the direct-to-LDS GEMM (one struct, passed by value).
struct GemmArgs {
  const void* x;  // W-only: fp16/bf16 activations; I8: s8 quantized activations
  int64_t ldx;    // row stride: elements (W-only) or bytes (I8)
  int M, Kc;
  const uint8_t* packed;
  const float* scale;
  const float* bias;
  const int32_t* colsum;  // I8 only
  int N, Nt;
  void* y;
  int yt;
  int64_t ldy;
  int32_t* acc_out;     // I8 only, may be null
  const float* qpbuf;   // I8 only: (s_x, zp as int bits)
  const float* rsum;    // fp16 W-only with RSP: per-row sums of x [M]
  const float* rscale;  // fp16 W-only with RSP, nullable: per-row output scale [M]
  int flags;            // bit 1: x rows vector loads; 2: y rows 4-element vector stores;
                        // 4: W8A8 per-token epilogue; 8: y and ldy 16-byte aligned
  // split K (gridDim.z > 1): partial tiles [tile][split] of dl_tile_bytes()
  // each, and one counter per output tile (zeroed by the pre-pass)
  uint8_t* part;
  uint32_t* tcount;
  int splits;
};

// KG groups of WN x WM waves: group kg streams the K tiles
// [kg*KW, kg*KW + KW), KW = ceil(Kc/KG), through its own NS-stage ring; the
// groups step in lockstep (one barrier per stage) and their partial tiles are
// summed through LDS in group order at the end.  Splitting K inside the
// workgroup multiplies the waves per SIMD (latency hiding) for grids too small
// to fill the chip, without extra HBM traffic.
// Bytes of the epilogue operand table: per block column its scale, bias and
// (W8A8) column sum, per block row its row sum and row scale, and the two
// activation quantization words.
constexpr int dl_epi_table_bytes(int BN, int BM) { return ((3 * BN + 2 * BM + 2) * 4 + 15) & ~15; }

// LDS bytes of one workgroup: the stage rings (or, after the K loop, the
// cross-group reduction buffer / the staged output tile), plus the in-loop row
// sums of fp16 W-only blocks without precomputed sums, plus the epilogue
// operand table where the stage bytes left free after the K loop cannot hold it.
template <bool I8, int XT, int BN, int BM, int WN, int WM, int NS, int KG, bool RSP, int KT>
constexpr int dl_lds_bytes() {
  const int stage = KT * ((BN / 16) * 1024 + BM * (I8 ? 64 : 128));
  const int red = (KG - 1) * WN * WM * (BN / WN / 16) * (BM / WM / 16) * 1024;
  const int ldsb = KG * NS * stage > red ? KG * NS * stage : red;
  const int epi = KG == 1 ? BM * (BN * 2 + 32) : 0;
  const int ldsa = epi > ldsb ? epi : ldsb;
  const bool rsk = !I8 && XT == XT_F16 && !RSP;
  const int post = KG == 1 ? epi : red;  // bytes from offset 0 in use after the K loop
  const int epb = dl_epi_table_bytes(BN, BM);
  return ldsa + (rsk ? KG * BM * 4 : 0) + (post + epb <= ldsa ? 0 : epb);
}
constexpr int kMaxLdsBytes = 160 * 1024;  // gfx950: LDS per workgroup (and per CU)
constexpr int kXCDs = 8;                  // MI355X: accelerator complex dies, each with its own L2

// Occupancy hint (waves per SIMD): what the LDS leaves room for, at most 4
// (128 VGPRs), or 2 (256 VGPRs) when a wave's accumulator tile exceeds 64 x 64.
// A workgroup's KG * WN * WM waves spread over the CU's 4 SIMDs, and
// kMaxLdsBytes / dl_lds_bytes workgroups fit a CU; asking for more waves
// than the LDS admits would only tighten the register budget.
template <bool I8, int XT, int BN, int BM, int WN, int WM, int NS, int KG, bool RSP, int KT>
constexpr int dl_min_waves() {
  const int regs = (BN / WN) * (BM / WM) > 64 * 64 ? 2 : 4;
  const int lds = kMaxLdsBytes / dl_lds_bytes<I8, XT, BN, BM, WN, WM, NS, KG, RSP, KT>() * KG * WN * WM / 4;
  return lds < 1 ? 1 : (lds < regs ? lds : regs);
}

// RSP (fp16 W-only): the per-row sums of x come precomputed in a.rsum instead
// of being accumulated in the K loop.
// KT (W8A8, one K group): K tiles per stage.  An i8 MFMA covers a whole 64-wide
// K tile, so a one-tile stage holds half the MFMAs of an fp16 stage per
// barrier; two tiles per stage restore the ratio.  Sub-stage j of a stage holds
// weight tiles and activation columns of K tile KT * stage + j, laid out as a
// one-tile stage.
// SK: K split over gridDim.z workgroups with the partial-tile fixup (only the
// configurations the split plan uses are built with it: the fixup's registers
// would otherwise spill in the large-tile configurations).  Its grids are
// small, so the occupancy hint asks for at most 2 waves per SIMD (256 VGPRs):
// the fixup holds every other split's partial tile in registers at once.
template <bool I8, int XT, int BN, int BM, int WN, int WM, int NS, int KG, bool RSP = false, int KT = 1, bool SK = false>
__global__ __launch_bounds__(KG* WN* WM * 64, (SK ? (dl_min_waves<I8, XT, BN, BM, WN, WM, NS, KG, RSP, KT>() < 2
                                                          ? dl_min_waves<I8, XT, BN, BM, WN, WM, NS, KG, RSP, KT>()
                                                          : 2)
                                                    : dl_min_waves<I8, XT, BN, BM, WN, WM, NS, KG, RSP, KT>())) void gemm_dl_kernel(const GemmArgs a) {
  typedef GemmOp<XT> Op;
  typedef typename Op::V V;
  typedef typename std::conditional<I8, i32x4, f32x4>::type Acc;
  constexpr int GW = WN * WM;
  constexpr int TN = BN / WN, TM = BM / WM, FN = TN / 16, FM = TM / 16;
  constexpr int XB = I8 ? 64 : 128;     // bytes of one activation row per stage
  constexpr int WT = BN / 16;           // weight tiles per stage
  constexpr int XR = BM * XB / 1024;    // 1 KiB activation chunks per stage
  constexpr int WBYTES = WT * 1024, SUB = WBYTES + BM * XB, STAGE = KT * SUB;
  constexpr int LPS = KT * (WT + XR) / GW;  // DMA instructions per wave per stage
  constexpr int RED = (KG - 1) * GW * FN * FM * 1024;
  constexpr int LDSB = KG * NS * STAGE > RED ? KG * NS * STAGE : RED;
  // fp16 activations: weights enter the MFMA as subnormals u * 2^-24 (u = q + 128,
  // one v_perm per pair); the 128 * rowsum(x) offset is removed in the epilogue.
  constexpr bool OFS = !I8 && XT == XT_F16;
  constexpr bool RSK = OFS && !RSP;  // row sums accumulated here
  constexpr int RF = FM / WN;        // activation fragments whose row sums each wave keeps
  static_assert(WT % GW == 0 && XR % GW == 0, "even DMA split");
  static_assert(NS >= 2 && NS <= 8, "stages");
  static_assert(FM % WN == 0, "row-sum split");
  static_assert(KT == 1 || (I8 && KG == 1), "K-tile pairs: W8A8 with one K group");
  // 2-byte outputs (fp16 / bf16) of one-group blocks leave through LDS: the
  // block's output tile is written there (rows padded by 32 bytes against bank
  // conflicts), then stored as whole 16-byte row chunks instead of 8-byte
  // pieces per lane (full cache lines; measured 3-6% on the fp16 GEMM).
  constexpr bool LEPI = KG == 1;
  constexpr int ERS = BN * 2 + 32;  // bytes per padded row of the LDS output tile
  constexpr int LDSA = (LEPI && BM * ERS > LDSB) ? BM * ERS : LDSB;
  // Epilogue operand table (EPB bytes at EPO): the stage bytes beyond the
  // output tile / reduction buffer when they are free after the K loop, else
  // appended after the in-loop row sums.
  constexpr int EPB = dl_epi_table_bytes(BN, BM);
  constexpr int POST = LEPI ? BM * ERS : RED;
  constexpr bool EPIN = POST + EPB <= LDSA;
  constexpr int EPO = EPIN ? LDSA - EPB : LDSA + (RSK ? KG * BM * 4 : 0);
  // one LDS object: with a second one the compiler waits for every stage DMA in
  // flight before any LDS read of the main loop (it cannot tell them apart)
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDSA + (RSK ? KG * BM * 4 : 0) + (EPIN ? 0 : EPB)];
  static_assert(sizeof(lds) == dl_lds_bytes<I8, XT, BN, BM, WN, WM, NS, KG, RSP, KT>(), "launcher's LDS model");
  float* const rsum_lds = (float*)(lds + LDSA);
  // table: scale [BN], bias [BN], column sums [BN] (int), row sums [BM], row
  // scales [BM], the two activation quantization words
  float* const ept = (float*)(lds + EPO);
  constexpr int EP_BI = BN, EP_CS = 2 * BN, EP_RS = 3 * BN, EP_RF = 3 * BN + BM, EP_QP = 3 * BN + 2 * BM;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r = lane & 15, g = lane >> 4;
  const int kg = wave / GW, w = __builtin_amdgcn_readfirstlane(wave % GW);  // wave-uniform: LDS targets stay scalar
  const int wn = w / WM, wm = w % WM;
  // Block order.  Workgroup L = x + gridDim.x * y runs on XCD L % 8, so when
  // the grid is a multiple of 8 blocks wide every row block of a weight
  // column block lands on one XCD and shares its L2.  Other widths would
  // spread each column block over the XCDs (its weights fetched into up to 8
  // L2s): there each XCD takes a contiguous column-major range of blocks
  // instead (measured: the fastest configuration 2.4% (fp16) / 4.0% (W8A8)
  // faster over 31 such shapes, up to 15%; no configuration more than 5% slower).
  int bx = blockIdx.x, by = blockIdx.y;
  if constexpr (!SK) {
    const int gx = gridDim.x;
    if (gx % kXCDs != 0) {  // 64-bit: gx * gridDim.y need not fit an int
      const int64_t gy = gridDim.y, T = gx * gy, L = bx + gx * (int64_t)by;
      const int64_t q = T / kXCDs, rr = T % kXCDs, xcd = L % kXCDs;
      const int64_t Lp = (xcd < rr ? xcd * (q + 1) : rr * (q + 1) + (xcd - rr) * q) + L / kXCDs;
      bx = (int)(Lp / gy);
      by = (int)(Lp - bx * gy);
    }
  }
  const int nt0 = bx * WT, m0 = by * BM;
  const int M = a.M, Kc = a.Kc, Nt = a.Nt;
  // stage steps of KT K tiles (the host keeps Kc % KT == 0)
  const int KX = Kc / KT;
  // split K over gridDim.z workgroups: split z takes stage steps [zb, zb + zc)
  // (the host keeps every split non-empty), its KG groups share them out
  const int S = SK ? (int)gridDim.z : 1, z = SK ? (int)blockIdx.z : 0;
  const int KXs = (KX + S - 1) / S;
  const int zb = z * KXs, zc = min(KXs, KX - zb);
  const int KW = (zc + KG - 1) / KG;
  const int kbeg = zb + kg * KW;
  const int cnt = min(KW, zb + zc - kbeg);  // tiles of this group (<= 0: none)
  const uint8_t* xg = (const uint8_t*)a.x;
  const int64_t xrow = I8 ? a.ldx : a.ldx * 2;  // bytes per activation row

  // Per-lane byte offsets of this wave's DMA slots from the block's first
  // weight tile / activation row; fixed over the K loop, so each stage issues
  // from a wave-uniform base (scalar registers) plus these offsets.  The
  // launcher keeps them below 2^31.
  uint32_t woff[WT / GW], xoff[XR / GW];
#pragma unroll
  for (int i2 = 0; i2 < WT / GW; ++i2) {
    const int j = w * (WT / GW) + i2;
    woff[i2] = (uint32_t)(min(nt0 + j, Nt - 1) - nt0) * (uint32_t)Kc * 1024u + lane * 16;
  }
#pragma unroll
  for (int i2 = 0; i2 < XR / GW; ++i2) {
    const int j = w * (XR / GW) + i2;
    if constexpr (I8) {
      const int row = j * 16 + (lane >> 2);
      const int chunk = (lane & 3) ^ ((row >> 2) & 3);
      xoff[i2] = (uint32_t)((int64_t)(min(m0 + row, M - 1) - m0) * xrow) + chunk * 16;
    } else {
      const int row = j * 8 + (lane >> 3);
      const int chunk = (lane & 7) ^ ((row >> 1) & 7);
      xoff[i2] = (uint32_t)((int64_t)(min(m0 + row, M - 1) - m0) * xrow) + chunk * 16;
    }
  }
  const __amdgpu_buffer_rsrc_t wrs =
      raw_rsrc(a.packed + (int64_t)nt0 * Kc * 1024, (uint32_t)min((int64_t)(Nt - nt0) * Kc * 1024, (int64_t)0xffffffff));
  const __amdgpu_buffer_rsrc_t xrs =
      raw_rsrc(xg + (int64_t)m0 * xrow, (uint32_t)min((int64_t)(M - m0) * xrow, (int64_t)0xffffffff));

  // this wave's LDS slots within a stage (scalar)
  const int wslot = __builtin_amdgcn_readfirstlane(w * (WT / GW) * 1024);
  const int xslot = __builtin_amdgcn_readfirstlane(WBYTES + w * (XR / GW) * 1024);
  auto issue = [&](int i, int st) {
    // clamped: the surplus stages of a short last group are never multiplied
    const int ks = KG == 1 ? zb + i : max(0, min(kbeg + min(i, cnt - 1), KX - 1));
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      const int kc = ks * KT + j;
      const int sb = __builtin_amdgcn_readfirstlane((kg * NS + st) * STAGE + j * SUB);
#pragma unroll
      for (int i2 = 0; i2 < WT / GW; ++i2) lds_dma16_buf(wrs, woff[i2], kc * 1024, lds + sb + wslot + i2 * 1024);
#pragma unroll
      for (int i2 = 0; i2 < XR / GW; ++i2)
        lds_dma16_buf(xrs, xoff[i2], kc * (I8 ? 64 : 128), lds + sb + xslot + i2 * 1024);
    }
  };

  Acc acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int b = 0; b < FM; ++b) acc[i][b] = Acc{0, 0, 0, 0};
  // OFS: wave (wn, wm) sums the activation rows of fragments b = wn + j*WN
  // (each row of the block once over the WN waves); lane (g, r) holds row r of
  // the fragment over its K columns
  float rs[RF];
#pragma unroll
  for (int j = 0; j < RF; ++j) rs[j] = 0.0f;

  // Epilogue operands, loaded before the first stage so that their latency
  // hides behind the K loop (loaded at its end they cost a full memory round
  // trip per block: 2-3.5 us of a 13 us small-M launch): thread t holds block
  // column min(t, BN-1) and block row min(t, BM-1), indexes clamped so every
  // load is unconditional.  They are the oldest loads in flight, so the first
  // stage wait covers them.
  constexpr int NTH = KG * GW * 64;
  static_assert(NTH >= BN && NTH >= BM, "one thread per block column and row");
  const bool ptok = I8 && (a.flags & 4);  // I8 per-token symmetric (flags bit 4)
  const int ecol = min(nt0 * 16 + min(tid, BN - 1), a.N - 1);
  const int erow = min(m0 + min(tid, BM - 1), M - 1);
  const float e_sc = a.scale[ecol];
  const float e_bi = a.bias ? a.bias[ecol] : -0.0f;  // -0: adding it changes no value
  int e_cs = 0;
  float e_q = 0.0f;
  if constexpr (I8) {
    if (!ptok) {
      e_cs = a.colsum[ecol];
      e_q = a.qpbuf[tid & 1];
    }
  }
  float e_rs = 0.0f, e_rf = 1.0f;
  if constexpr (OFS && !RSK) e_rs = a.rsum[erow];
  if constexpr (RSP || I8)
    if (a.rscale) e_rf = a.rscale[erow];

#pragma unroll
  for (int i = 0; i < NS - 1; ++i)
    if (i < KW) issue(i, i);
  for (int i = 0; i < KW; ++i) {
    // stage i has landed once only the younger in-flight stages remain
    wait_stages<LPS, NS>(min(NS - 2, KW - 1 - i));
    barrier_nofence();
    if (i + NS - 1 < KW) issue(i + NS - 1, (i + NS - 1) % NS);
    if (KG == 1 || i < cnt) {
      const uint8_t* wb = lds + (kg * NS + i % NS) * STAGE;
      const uint8_t* xs = wb + WBYTES;
      if constexpr (I8) {
#pragma unroll
        for (int j = 0; j < KT; ++j) {
          i32x4 xf[FM];
#pragma unroll
          for (int b = 0; b < FM; ++b) xf[b] = *(const i32x4*)(xs + j * SUB + xq_off(wm * TM + b * 16 + r, g));
#pragma unroll
          for (int t = 0; t < FN; ++t) {
            const i32x4 wf = tile_to_s8(*(const u32x4*)(wb + j * SUB + (wn * FN + t) * 1024 + lane * 16));
#pragma unroll
            for (int b = 0; b < FM; ++b)
              acc[t][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf, xf[b], acc[t][b], 0, 0, 0);
          }
        }
      } else {
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          V xf[FM];
#pragma unroll
          for (int b = 0; b < FM; ++b) xf[b] = *(const V*)(xs + xsw_off(wm * TM + b * 16 + r, 2 * g + s2));
          if constexpr (RSK) {
#pragma unroll
            for (int j = 0; j < RF; ++j) {
              const u32x4 xv = *(const u32x4*)(xs + xsw_off(wm * TM + (wn + j * WN) * 16 + r, 2 * g + s2));
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const uint32_t word = xv[e];  // bit_cast of a vector element reads element 0: copy first
                rs[j] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, word), (f16x2){1.0f16, 1.0f16}, rs[j], false);
              }
            }
          }
#pragma unroll
          for (int t = 0; t < FN; ++t) {
            const u32x2 raw = *(const u32x2*)(wb + (wn * FN + t) * 1024 + lane * 16 + s2 * 8);
            V wf0, wf1;
            if constexpr (OFS)
              wf0 = u8x8_to_f16_sub(raw.x, raw.y);
            else
              Op::wconv((u32x4){raw.x, raw.y, 0u, 0u}, wf0, wf1);
#pragma unroll
            for (int b = 0; b < FM; ++b) acc[t][b] = Op::mma(wf0, xf[b], acc[t][b]);
          }
        }
      }
    }
    // No barrier here: the stage this step read is overwritten only by the
    // issue after the next step's barrier, which every wave reaches after its
    // reads of this stage have returned (their MFMAs consumed them).
  }

  // Every wave is past its last stage (its final wait was vmcnt(0)) and its
  // LDS reads have returned: the epilogue operands move into their table.
  __syncthreads();
  if (tid < BN) {
    ept[tid] = e_sc;
    ept[EP_BI + tid] = e_bi;
    ((int*)ept)[EP_CS + tid] = e_cs;
  }
  if (tid < BM) {
    ept[EP_RS + tid] = e_rs;
    ept[EP_RF + tid] = e_rf;
  }
  if (tid < 2) ept[EP_QP + tid] = e_q;
  __syncthreads();

  if constexpr (RSK) {
    // sum the 4 K-column groups of each row, then publish the block's row sums
#pragma unroll
    for (int j = 0; j < RF; ++j) {
      rs[j] += __shfl_xor(rs[j], 16);
      rs[j] += __shfl_xor(rs[j], 32);
      if (g == 0) rsum_lds[kg * BM + wm * TM + (wn + j * WN) * 16 + r] = rs[j];
    }
    if constexpr (KG == 1) __syncthreads();  // every stage has landed: the fence costs nothing here
  }
  if constexpr (KG > 1) {
    barrier_nofence();  // every group is done with its stages before they become the reduction buffer
    Acc* red = (Acc*)lds;
    if (kg > 0) {
#pragma unroll
      for (int t = 0; t < FN; ++t)
#pragma unroll
        for (int b = 0; b < FM; ++b) red[(((kg - 1) * GW + w) * FN * FM + t * FM + b) * 64 + lane] = acc[t][b];
    }
    __syncthreads();  // no DMA is in flight any more: the fence costs nothing here
    if (kg > 0) return;
#pragma unroll 1
    for (int k = 1; k < KG; ++k)
#pragma unroll
      for (int t = 0; t < FN; ++t)
#pragma unroll
        for (int b = 0; b < FM; ++b) acc[t][b] += red[(((k - 1) * GW + w) * FN * FM + t * FM + b) * 64 + lane];
  }

  if constexpr (SK) {
    // Split K: store this split's partial tile (device-coherent stores), then
    // count the tile's splits; the last split to arrive adds every split's
    // partial in split order (the same fp32 sum whichever split is last) and
    // runs the epilogue.  Each wave waits for its stores (vmcnt 0) before the
    // workgroup's count is issued, so a count implies the partial is in
    // place; the last split's loads are issued after its count returned.
    constexpr uint32_t kTile = GW * FN * FM * 1024;  // bytes of one partial tile
    const int tile = blockIdx.y * gridDim.x + blockIdx.x;
    const __amdgpu_buffer_rsrc_t prs = raw_rsrc(a.part + (size_t)tile * S * kTile, S * kTile);
    const uint32_t mine = (uint32_t)(w * FN * FM) * 1024u + lane * 16u;
#pragma unroll
    for (int t = 0; t < FN; ++t)
#pragma unroll
      for (int b = 0; b < FM; ++b)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[t][b]), prs,
                                               z * kTile + mine + (t * FM + b) * 1024, 0, kCoherent);
    wait_vmcnt<0>();
    __syncthreads();  // every wave's partial stores are performed
    uint32_t* const flag = (uint32_t*)lds;
    if (w == 0 && lane == 0)
      *flag = __hip_atomic_fetch_add(a.tcount + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const uint32_t arrived = *flag;
    if (arrived != (uint32_t)S - 1) return;
    // every split of the tile has counted: leave the counter at zero (the
    // pre-pass zeroes it too, for a workspace that holds anything)
    if (w == 0 && lane == 0) __hip_atomic_store(a.tcount + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // The other splits' partials, all in flight at once (one memory round
    // trip; loading them split by split cost one round trip each: 4.6 us on
    // the last split of a 4-way M = 128 tile), then summed in split order
    // 0 .. S-1 with this split's own partial at z, so the sum has the same
    // bits whichever split arrives last.
    static_assert(kMaxSplits == 4, "the partial slots below");
    u32x4 v[kMaxSplits][FN][FM];
#pragma unroll
    for (int zz = 0; zz < kMaxSplits; ++zz) {
#pragma unroll
      for (int t = 0; t < FN; ++t)
#pragma unroll
        for (int b = 0; b < FM; ++b)
          v[zz][t][b] = zz < S && zz != z  // uniform
                            ? __builtin_amdgcn_raw_buffer_load_b128(prs, zz * kTile + mine + (t * FM + b) * 1024, 0,
                                                                    kCoherent)
                            : (u32x4){0u, 0u, 0u, 0u};
    }
    Acc sum[FN][FM];
#pragma unroll
    for (int t = 0; t < FN; ++t)
#pragma unroll
      for (int b = 0; b < FM; ++b) sum[t][b] = Acc{0, 0, 0, 0};
#pragma unroll
    for (int zz = 0; zz < kMaxSplits; ++zz) {
      if (zz < S) {  // uniform
        const bool own = zz == z;
#pragma unroll
        for (int t = 0; t < FN; ++t)
#pragma unroll
          for (int b = 0; b < FM; ++b) sum[t][b] += own ? acc[t][b] : __builtin_bit_cast(Acc, v[zz][t][b]);
      }
    }
#pragma unroll
    for (int t = 0; t < FN; ++t)
#pragma unroll
      for (int b = 0; b < FM; ++b) acc[t][b] = sum[t][b];
    __syncthreads();  // the flag's LDS word is free again (the staged epilogue below reuses it)
  }

  const bool yvec = a.flags & 2;
  // I8 per-token symmetric (ptok): no zero point, y = fp32(acc) * fp32(s_t[m] * scale[n])
  // every wave is past the K loop and no stage DMA is in flight (the last wait
  // was vmcnt(0)): the stage buffers become the output tile
  const bool lepi = LEPI && a.yt != XT_F32;
  if (lepi) __syncthreads();
  float sx = 0.0f;
  int corr = 0;
  if constexpr (I8) {
    if (!ptok) {
      sx = ept[EP_QP];
      corr = 128 - __float_as_int(ept[EP_QP + 1]);
    }
  }
  // Straight-line epilogue: every table entry is valid (rows >= M and columns
  // >= N hold the last row / column, and are never stored), a missing bias is
  // -0 (x + -0 and fma(x, f, -0) equal x and x * f bit for bit) and a missing
  // row scale 1, so no operand read or output value depends on a branch.
  // OFS: acc = 2^-24 * sum (q + 128) x, so y = (acc - 2^-17 * rowsum) * (scale * 2^24)
  // (* rscale[m] for staged fp32 / bf16 activations)
  float rc[FM], rf[FM];
#pragma unroll
  for (int b = 0; b < FM; ++b) {
    const int rl = wm * TM + b * 16 + r;  // block row of the table
    rc[b] = 0.0f;
    rf[b] = RSP || I8 ? ept[EP_RF + rl] : 1.0f;
    if constexpr (RSK) {
      float t2 = 0.0f;
#pragma unroll
      for (int k = 0; k < KG; ++k) t2 += rsum_lds[k * BM + rl];
      rc[b] = t2 * 0x1p-17f;
    } else if constexpr (OFS) {
      rc[b] = ept[EP_RS + rl] * 0x1p-17f;
    }
  }
  // per-column operands of wave tile column t (lane columns cl0 .. cl0 + 3)
  auto col_ops = [&](int t, f32x4& sc, f32x4& bi, i32x4& cs) {
    const int cl0 = (wn * FN + t) * 16 + 4 * g;
    const f32x4 scv = *(const f32x4*)(ept + cl0);
    bi = *(const f32x4*)(ept + EP_BI + cl0);
    cs = (i32x4){0, 0, 0, 0};
    if constexpr (I8) cs = *(const i32x4*)(ept + EP_CS + cl0);
#pragma unroll
    for (int v = 0; v < 4; ++v) sc[v] = I8 ? (ptok ? scv[v] : sx * scv[v]) : (OFS ? scv[v] * 0x1p24f : scv[v]);
  };
  auto out4 = [&](int t, int b, const f32x4& sc, const f32x4& bi, const i32x4& cs) {
    f32x4 o;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if constexpr (I8) {
        const int av = acc[t][b][v] + corr * cs[v];
        const float f = ptok ? rf[b] * sc[v] : sc[v];
        o[v] = __builtin_fmaf((float)av, f, bi[v]);
      } else {
        const float out = OFS ? ((acc[t][b][v] - rc[b]) * sc[v]) * rf[b] : acc[t][b][v] * sc[v];
        o[v] = out + bi[v];
      }
    }
    return o;
  };
  // the whole tile into LDS (rows >= M / columns >= N are never copied out),
  // one straight loop per output type
  auto tile_to_lds = [&](auto f16y) {
#pragma unroll
    for (int t = 0; t < FN; ++t) {
      f32x4 sc, bi;
      i32x4 cs;
      col_ops(t, sc, bi, cs);
#pragma unroll
      for (int b = 0; b < FM; ++b) {
        const f32x4 o = out4(t, b, sc, bi, cs);
        uint32_t lo, hi;
        if constexpr (decltype(f16y)::value) {
          lo = pack_h2(out_f16(o[0]), out_f16(o[1]));
          hi = pack_h2(out_f16(o[2]), out_f16(o[3]));
        } else {
          lo = pack_b2(out_bf16(o[0]), out_bf16(o[1]));
          hi = pack_b2(out_bf16(o[2]), out_bf16(o[3]));
        }
        *(u32x2*)(lds + (wm * TM + b * 16 + r) * ERS + ((wn * FN + t) * 16 + 4 * g) * 2) = (u32x2){lo, hi};
      }
    }
  };
  if (lepi) {
    if (a.yt == XT_F16)
      tile_to_lds(std::true_type{});
    else
      tile_to_lds(std::false_type{});
  } else {
#pragma unroll
    for (int t = 0; t < FN; ++t) {
      const int n = (nt0 + wn * FN + t) * 16 + 4 * g;
      const int nvalid = min(4, a.N - n);
      f32x4 sc, bi;
      i32x4 cs;
      col_ops(t, sc, bi, cs);
#pragma unroll
      for (int b = 0; b < FM; ++b) {
        const int m = m0 + wm * TM + b * 16 + r;
        const f32x4 o = out4(t, b, sc, bi, cs);
        if (m < M && n < a.N) store_y4(a.y, a.yt, (int64_t)m * a.ldy + n, o, yvec && nvalid == 4, nvalid);
      }
    }
  }
  if constexpr (I8) {
    if (a.acc_out) {  // int32 accumulators with the zero-point correction (tests and tools)
#pragma unroll
      for (int t = 0; t < FN; ++t) {
        const int cl0 = (wn * FN + t) * 16 + 4 * g;
        const int n = nt0 * 16 + cl0;
        const i32x4 cs = *(const i32x4*)(ept + EP_CS + cl0);
#pragma unroll
        for (int b = 0; b < FM; ++b) {
          const int m = m0 + wm * TM + b * 16 + r;
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if (m < M && n + v < a.N) a.acc_out[(int64_t)m * a.N + n + v] = acc[t][b][v] + corr * cs[v];
        }
      }
    }
  }
  if constexpr (LEPI) {
    if (!lepi) return;
    __syncthreads();
    constexpr int CPR = BN * 2 / 16;  // 16-byte chunks per output row of the block
    constexpr int NT = WN * WM * 64;
    static_assert((BM * CPR) % NT == 0, "output chunks split evenly over the threads");
    const bool y16 = a.flags & 8;  // y and its row stride 16-byte aligned
    uint16_t* const y2 = (uint16_t*)a.y;
#pragma unroll
    for (int p = 0; p < BM * CPR / NT; ++p) {
      const int c = p * NT + tid;
      const int ml = c / CPR, ch = c - ml * CPR;
      const int m = m0 + ml, n = nt0 * 16 + ch * 8;
      if (m >= M || n >= a.N) continue;
      const u32x4 v = *(const u32x4*)(lds + ml * ERS + ch * 16);
      uint16_t* const yp = y2 + (int64_t)m * a.ldy + n;
      if (y16 && n + 8 <= a.N) {
        *(u32x4*)yp = v;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t word = v[e >> 1];
          if (n + e < a.N) yp[e] = (uint16_t)((e & 1) ? word >> 16 : word);
        }
      }
    }
  }
}

template <bool I8, int XT, int BN, int BM, int WN, int WM, int NS, int KG, bool RSP = false, int KT = 1, bool SK = false>
int launch_dl(const GemmArgs& a, hipStream_t st) {
  if constexpr (dl_lds_bytes<I8, XT, BN, BM, WN, WM, NS, KG, RSP, KT>() > kMaxLdsBytes) {
    return -1;  // no such kernel: its LDS would not fit (the pickers never ask for it)
  } else {
    if (a.Kc % KT) return -1;
    if (SK != (a.part != nullptr)) return -1;  // split arguments only for the split instances
    if (SK && (a.splits < 2 || a.splits > kMaxSplits)) return -1;
    const dim3 grid((unsigned)((a.Nt + BN / 16 - 1) / (BN / 16)), (unsigned)((a.M + BM - 1) / BM),
                    (unsigned)(SK ? a.splits : 1));
    hipLaunchKernelGGL((gemm_dl_kernel<I8, XT, BN, BM, WN, WM, NS, KG, RSP, KT, SK>), grid, dim3(KG * WN * WM * 64),
                       0, st, a);
    return check_launch();
  }
}

// ---------------------------------------------------------------------------
// W8A8 prefill: the activations are quantized once, into the caller's
// workspace, as s8 (xq - 128) rows of Kp = Kc*64 bytes (columns >= K are 0 and
// meet zero weights); gemm_w8a8_dl_kernel then runs the direct-to-LDS
// pipeline on s8 operands with v_mfma_i32_16x16x64_i8.
// ---------------------------------------------------------------------------
// VEC: 16-byte aligned rows and K % 16 == 0 (every chunk is whole, branch-free loads).
// QC: 16-element chunks per thread (1 for small x, so that the grid still
// covers every CU).
template <int XT, bool VEC, int QC>
__global__ __launch_bounds__(256) void quantize_act_kernel(const void* __restrict__ x, int64_t ldx, int M, int K,
                                                           int Kp, const float2* __restrict__ partials, int nparts,
                                                           int8_t* __restrict__ xq, float* __restrict__ qp_out,
                                                           int flags) {
  // QC 16-element chunks per thread, chunk i of the block at
  // (block * QC + i) * 256 + thread.  The activation loads go out
  // first; the (latency-bound) reduction of the partials and fbgemm's
  // double-precision parameter choice run while they are in flight.
  const int cpr = Kp / 16;
  const int64_t nch = (int64_t)M * cpr;
  float t[QC][16];
  int64_t cc[QC];
#pragma unroll
  for (int i = 0; i < QC; ++i) {
    cc[i] = ((int64_t)blockIdx.x * QC + i) * blockDim.x + threadIdx.x;
    const int64_t c = min(cc[i], nch - 1);  // clamped: surplus chunks are loaded but not stored
    const int m = (int)(c / cpr), k0 = (int)(c - (int64_t)m * cpr) * 16;
    if constexpr (VEC) {
      typedef typename XElem<XT>::T T;
      typedef T v8 __attribute__((ext_vector_type(8)));
      // K % 16 == 0: a chunk is either inside the row or wholly in the
      // padding columns K..Kp-1, whose values are never used (they quantize
      // to s8 0 below); padding chunks load the row's last chunk instead of
      // reading past the row (past the end of x on the last row)
      const T* p = (const T*)x + act_chunk_src(c, cpr, K, ldx);
      if constexpr (XT == XT_F32) {
        const f32x4 a0 = *(const f32x4*)p, a1 = *(const f32x4*)(p + 4);
        const f32x4 a2 = *(const f32x4*)(p + 8), a3 = *(const f32x4*)(p + 12);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          t[i][j] = a0[j];
          t[i][4 + j] = a1[j];
          t[i][8 + j] = a2[j];
          t[i][12 + j] = a3[j];
        }
      } else {
        const v8 a0 = *(const v8*)p, a1 = *(const v8*)(p + 8);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          t[i][j] = XElem<XT>::to_f32(a0[j]);
          t[i][8 + j] = XElem<XT>::to_f32(a1[j]);
        }
      }
    } else {
      load8_f32<XT>(x, ldx, M, K, m, k0, flags & 1, t[i]);
      load8_f32<XT>(x, ldx, M, K, m, k0 + 8, flags & 1, t[i] + 8);
    }
  }
  __shared__ float red[16];
  const ActQParams qp = block_qparams_from_partials(partials, nparts, red);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    qp_out[0] = qp.scale;
    qp_out[1] = __int_as_float(qp.zp);
  }
#pragma unroll
  for (int i = 0; i < QC; ++i) {
    if (cc[i] >= nch) break;
    const int m = (int)(cc[i] / cpr), k0 = (int)(cc[i] - (int64_t)m * cpr) * 16;
    uint32_t d[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float u[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int jj = 4 * w + j;
        u[j] = k0 + jj < K ? __builtin_fmaf(t[i][jj], qp.inv, qp.zpf) : 128.0f;  // padding columns: s8 0
      }
      d[w] = pack_act_s8x4(u[0], u[1], u[2], u[3]);
    }
    *(u32x4*)(xq + (int64_t)m * Kp + k0) = (u32x4){d[0], d[1], d[2], d[3]};
  }
}


// Dense x (ldx == K, 16-byte aligned) with K % 64 == 0: the rows of x and of
// xq (Kp == K) are one flat array each, so chunk c of 16 values goes from
// x + 16c to xq + 16c with no division or padding.  QC chunks per thread, at
// (block * QC + i) * 256 + thread; loads clamped to the last chunk, stores
// guarded.
template <int XT, int QC>
__global__ __launch_bounds__(256) void quantize_dense_kernel(const void* __restrict__ x, int64_t nch,
                                                             const float2* __restrict__ partials, int nparts,
                                                             int8_t* __restrict__ xq, float* __restrict__ qp_out) {
  typedef typename XElem<XT>::T T;
  typedef T v8 __attribute__((ext_vector_type(8)));
  float t[QC][16];
  int64_t cc[QC];
#pragma unroll
  for (int i = 0; i < QC; ++i) {
    cc[i] = ((int64_t)blockIdx.x * QC + i) * blockDim.x + threadIdx.x;
    const T* p = (const T*)x + min(cc[i], nch - 1) * 16;
    if constexpr (XT == XT_F32) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 a = *(const f32x4*)(p + 4 * q);
#pragma unroll
        for (int j = 0; j < 4; ++j) t[i][4 * q + j] = a[j];
      }
    } else {
      const v8 a0 = *(const v8*)p, a1 = *(const v8*)(p + 8);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        t[i][j] = XElem<XT>::to_f32(a0[j]);
        t[i][8 + j] = XElem<XT>::to_f32(a1[j]);
      }
    }
  }
  __shared__ float red[16];
  const ActQParams qp = block_qparams_from_partials(partials, nparts, red);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    qp_out[0] = qp.scale;
    qp_out[1] = __int_as_float(qp.zp);
  }
#pragma unroll
  for (int i = 0; i < QC; ++i) {
    uint32_t d[4];
#pragma unroll
    for (int w = 0; w < 4; ++w)
      d[w] = pack_act_s8x4(__builtin_fmaf(t[i][4 * w], qp.inv, qp.zpf), __builtin_fmaf(t[i][4 * w + 1], qp.inv, qp.zpf),
                           __builtin_fmaf(t[i][4 * w + 2], qp.inv, qp.zpf),
                           __builtin_fmaf(t[i][4 * w + 3], qp.inv, qp.zpf));
    if (cc[i] < nch) *(u32x4*)(xq + cc[i] * 16) = (u32x4){d[0], d[1], d[2], d[3]};
  }
}

// Direct-to-LDS configurations (BN, BM, WN, WM, NS, KG), indexed by id.
#define SBQ_DL_CONFIGS(X) \
  X(0, 256, 128, 4, 2, 2, 1) \
  X(1, 256, 128, 4, 2, 3, 1) \
  X(2, 128, 128, 2, 2, 2, 1) \
  X(3, 128, 64, 2, 2, 2, 1)  \
  X(4, 128, 64, 2, 2, 2, 2)  \
  X(5, 128, 64, 2, 2, 2, 4)  \
  X(6, 128, 128, 2, 2, 2, 2) \
  X(7, 256, 128, 4, 2, 2, 2) \
  X(8, 64, 64, 1, 2, 2, 4)   \
  X(9, 128, 64, 2, 2, 3, 2)  \
  X(10, 256, 128, 4, 1, 2, 1) \
  X(11, 128, 256, 2, 2, 2, 1) \
  X(12, 256, 256, 4, 2, 2, 1) \
  X(16, 192, 64, 4, 1, 2, 1)  \
  X(17, 192, 64, 4, 1, 2, 4)  \
  X(18, 192, 128, 4, 1, 2, 1) \
  X(19, 192, 128, 4, 1, 3, 1) \
  X(22, 64, 64, 4, 1, 3, 1)

// The mid-sized-M configurations (64 weight rows, one 16-row tile per wave,
// every token of the block in each wave): (id, BM, NS).  They are built with
// precomputed row sums (fp16 W-only), two K tiles per stage (W8A8) and the
// split-K fixup as well.  Measured and not kept: 64 x 128 blocks (3 and 5
// stages) and 64 x 64 blocks with 5 and 8 stages (deeper rings were no faster:
// the ring's depth is not what bounds these shapes).
#define SBQ_MID_CONFIGS(X) \
  X(22, 64, 3)

template <bool I8, int XT>
int launch_dl_id(int id, const GemmArgs& a, hipStream_t st) {
  switch (id) {
#define SBQ_DL_CASE(ID, BN, BM, WN, WM, NS, KG) \
  case ID: return launch_dl<I8, XT, BN, BM, WN, WM, NS, KG>(a, st);
    SBQ_DL_CONFIGS(SBQ_DL_CASE)
#undef SBQ_DL_CASE
  }
  return -1;
}

// fp16 W-only with precomputed row sums: the configurations pick_gemm_dl
// chooses for W-only (the others run with the sums accumulated in the loop).
int launch_dl_rsp(int id, const GemmArgs& a, hipStream_t st) {
  switch (id) {
    case 0: return launch_dl<false, XT_F16, 256, 128, 4, 2, 2, 1, true>(a, st);
    case 2: return launch_dl<false, XT_F16, 128, 128, 2, 2, 2, 1, true>(a, st);
    case 3: return launch_dl<false, XT_F16, 128, 64, 2, 2, 2, 1, true>(a, st);
    case 5: return launch_dl<false, XT_F16, 128, 64, 2, 2, 2, 4, true>(a, st);
    case 8: return launch_dl<false, XT_F16, 64, 64, 1, 2, 2, 4, true>(a, st);
    case 10: return launch_dl<false, XT_F16, 256, 128, 4, 1, 2, 1, true>(a, st);
    case 16: return launch_dl<false, XT_F16, 192, 64, 4, 1, 2, 1, true>(a, st);
    case 17: return launch_dl<false, XT_F16, 192, 64, 4, 1, 2, 4, true>(a, st);
    case 18: return launch_dl<false, XT_F16, 192, 128, 4, 1, 2, 1, true>(a, st);
#define SBQ_MID_RSP(ID, BM, NS) \
    case ID: return launch_dl<false, XT_F16, 64, BM, 4, 1, NS, 1, true>(a, st);
    SBQ_MID_CONFIGS(SBQ_MID_RSP)
#undef SBQ_MID_RSP
  }
  if (a.rscale) return -1;  // staged activations need the row scale: only the configurations above apply it
  GemmArgs b = a;
  b.rsum = nullptr;
  return launch_dl_id<false, XT_F16>(id, b, st);
}

// W8A8 configurations with two K tiles per stage (ids 13-15, 20); an odd number
// of K tiles takes the one-tile configuration of the same block shape.
int launch_dl_i8(int id, const GemmArgs& a, hipStream_t st) {
  const bool kt2 = a.Kc % 2 == 0;
  switch (id) {
    case 13:
      return kt2 ? launch_dl<true, XT_F16, 256, 256, 4, 2, 2, 1, false, 2>(a, st) : launch_dl_id<true, XT_F16>(12, a, st);
    case 14:
      return kt2 ? launch_dl<true, XT_F16, 128, 128, 2, 2, 2, 1, false, 2>(a, st) : launch_dl_id<true, XT_F16>(2, a, st);
    case 15:
      return kt2 ? launch_dl<true, XT_F16, 128, 64, 2, 2, 2, 1, false, 2>(a, st) : launch_dl_id<true, XT_F16>(3, a, st);
    case 20:
      return kt2 ? launch_dl<true, XT_F16, 192, 64, 4, 1, 2, 1, false, 2>(a, st) : launch_dl_id<true, XT_F16>(16, a, st);
#define SBQ_MID_I8(ID, BM, NS) \
    case ID:                     \
      return kt2 ? launch_dl<true, XT_F16, 64, BM, 4, 1, NS, 1, false, 2>(a, st) : launch_dl_id<true, XT_F16>(ID, a, st);
    SBQ_MID_CONFIGS(SBQ_MID_I8)
#undef SBQ_MID_I8
  }
  return launch_dl_id<true, XT_F16>(id, a, st);
}

// The split-K instances: 128 x 64 blocks (ids 15 and 3, used by the tuning
// harness) and the mid-sized-M configurations.
int launch_dl_split(int id, bool i8, const GemmArgs& a, hipStream_t st) {
  const bool kt2 = a.Kc % 2 == 0;
  if (i8) {
    switch (id) {
      case 3:
      case 15:
        return kt2 ? launch_dl<true, XT_F16, 128, 64, 2, 2, 2, 1, false, 2, true>(a, st)
                   : launch_dl<true, XT_F16, 128, 64, 2, 2, 2, 1, false, 1, true>(a, st);
#define SBQ_MID_SPLIT_I8(ID, BM, NS)                                                \
      case ID:                                                                      \
        return kt2 ? launch_dl<true, XT_F16, 64, BM, 4, 1, NS, 1, false, 2, true>(a, st) \
                   : launch_dl<true, XT_F16, 64, BM, 4, 1, NS, 1, false, 1, true>(a, st);
      SBQ_MID_CONFIGS(SBQ_MID_SPLIT_I8)
#undef SBQ_MID_SPLIT_I8
    }
    return -1;
  }
  if (!a.rsum) return -1;  // fp16 W-only splits need the precomputed row sums
  switch (id) {
    case 3:
    case 15: return launch_dl<false, XT_F16, 128, 64, 2, 2, 2, 1, true, 1, true>(a, st);
#define SBQ_MID_SPLIT(ID, BM, NS) \
    case ID: return launch_dl<false, XT_F16, 64, BM, 4, 1, NS, 1, true, 1, true>(a, st);
    SBQ_MID_CONFIGS(SBQ_MID_SPLIT)
#undef SBQ_MID_SPLIT
  }
  return -1;
}

// Launch of direct-to-LDS configuration `id` (tuning entry; -1: no such id).
// Arguments with a split-K area (a.part) run the split instances.
int launch_gemm_dl_cfg(int id, bool i8, int xt, const GemmArgs& a, hipStream_t st) {
  if (a.part) return i8 || xt == XT_F16 ? launch_dl_split(id, i8, a, st) : -1;
  if (i8) return launch_dl_i8(id, a, st);
  // 192 x 64 blocks with K split over 4 wave groups leave no LDS for the
  // in-loop row sums: without precomputed sums the 128 x 64 split runs
  if (xt == XT_F16) return a.rsum ? launch_dl_rsp(id, a, st) : launch_dl_id<false, XT_F16>(id == 17 ? 5 : id, a, st);
  if (xt == XT_BF16) return launch_dl_id<false, XT_BF16>(id, a, st);
  return -2;
}

constexpr int64_t kCUs = 256;  // MI355X compute units

// Kernel-time model of one configuration (M > 128): its grid of G workgroups
// puts B = ceil(G / 256) on the busiest CU, which runs them in rounds of up to
// `occ` at once (occ: what LDS and registers admit per CU).  A round with j
// workgroups costs round[j-1] us per 64-wide K tile, and the kernel time is the
// busiest CU's rounds plus kc * Kc + c0.  The coefficients are least-squares
// fits (relative error) to GEMM-alone timings of every configuration on
// MI355X over 255 shapes: M = 192 .. 4096 (17 values) by N = 2048 .. 24576
// (11 values, 18820 among them) at K = 4096, and by N = 2048 .. 8192 at
// K = 12288.  Median error of the fitted times: 3.4% (fp16) / 3.5% (W8A8).
// Picking the smallest predicted time costs 0.1% (fp16) / 0.6% (W8A8) over the
// sum of those shapes against the fastest configuration of each, worst shape
// 1.06x / 1.17x (fitted on half of the shapes, it picks the other half within
// 0.1% / 0.7%).  The t256 ranges it replaced cost 3.4% / 9.2% there, with 17 /
// 42 shapes beyond 1.2x (W8A8 M = 640, N = 24576: 107.8 -> 64.1 us; fp16
// M = 1536, N = 8192: 118.4 -> 83.9 us).
struct PickCost {
  int id, wt, bm, occ;  // configuration, weight tiles (BN / 16) and rows per block, workgroups per CU
  float round[4], kc, c0;
};
constexpr PickCost kPickF16[] = {
    {0, 16, 128, 2, {0.8752f, 1.4950f, 0.0f, 0.0f}, -0.1906f, 7.419f},
    {2, 8, 128, 3, {0.5755f, 0.8307f, 1.2199f, 0.0f}, -0.0736f, 5.284f},
    {3, 8, 64, 4, {0.4421f, 0.4948f, 0.7084f, 0.9441f}, -0.0194f, 3.905f},
    {5, 8, 64, 1, {0.3427f, 0.0f, 0.0f, 0.0f}, -0.1125f, 8.834f},
    {8, 4, 64, 1, {0.2727f, 0.0f, 0.0f, 0.0f}, -0.1025f, 7.759f},
    {10, 16, 128, 2, {0.9332f, 1.5313f, 0.0f, 0.0f}, -0.1631f, 8.066f},
    {16, 12, 64, 4, {0.5219f, 0.6684f, 0.9792f, 1.2787f}, -0.0636f, 5.479f},
    {17, 12, 64, 1, {0.4311f, 0.0f, 0.0f, 0.0f}, -0.1362f, 9.805f},
    {18, 12, 128, 2, {0.8151f, 1.1780f, 0.0f, 0.0f}, -0.1713f, 8.224f},
};
constexpr PickCost kPickI8[] = {
    {0, 16, 128, 2, {0.6566f, 0.9437f, 0.0f, 0.0f}, -0.1356f, 5.191f},
    {1, 16, 128, 2, {0.6630f, 0.9696f, 0.0f, 0.0f}, -0.1773f, 7.038f},
    {2, 8, 128, 4, {0.4266f, 0.5184f, 0.7281f, 1.1083f}, 0.0164f, 1.486f},
    {3, 8, 64, 4, {0.4108f, 0.5000f, 0.5503f, 0.7116f}, -0.0362f, 0.290f},
    {8, 4, 64, 2, {0.2242f, 0.2806f, 0.0f, 0.0f}, -0.0666f, 6.374f},
    {12, 16, 256, 1, {0.9305f, 0.0f, 0.0f, 0.0f}, -0.2353f, 9.484f},
    {13, 16, 256, 1, {0.9188f, 0.0f, 0.0f, 0.0f}, -0.2204f, 9.060f},
    {14, 8, 128, 2, {0.3916f, 0.5393f, 0.0f, 0.0f}, -0.0723f, 5.289f},
    {15, 8, 64, 3, {0.2710f, 0.3348f, 0.5245f, 0.0f}, -0.0161f, 3.097f},
    {16, 12, 64, 4, {0.4147f, 0.4938f, 0.5822f, 0.9175f}, 0.0121f, 1.729f},
    {18, 12, 128, 2, {0.6125f, 0.7382f, 0.0f, 0.0f}, -0.1509f, 6.635f},
    {19, 12, 128, 2, {0.5758f, 0.7368f, 0.0f, 0.0f}, -0.1529f, 7.688f},
    {20, 12, 64, 2, {0.3710f, 0.4474f, 0.0f, 0.0f}, -0.0664f, 4.588f},
};

template <int N>
static int model_pick(const PickCost (&tab)[N], int64_t M, int64_t Nt, int64_t Kc) {
  int best = tab[0].id;
  double best_t = 0.0;
  for (int i = 0; i < N; ++i) {
    const PickCost& c = tab[i];
    const int64_t G = ((Nt + c.wt - 1) / c.wt) * ((M + c.bm - 1) / c.bm);
    const int64_t B = (G + kCUs - 1) / kCUs;  // workgroups on the busiest CU
    const int64_t full = B / c.occ, rem = B % c.occ;
    const double k = (double)Kc;
    const double t = (double)full * c.round[c.occ - 1] * k + (rem ? c.round[rem - 1] * k : 0.0) + c.kc * k + c.c0;
    if (i == 0 || t < best_t) {
      best = c.id;
      best_t = t;
    }
  }
  return best;
}

// Configuration for a shape.  M > 128 (fp16 W-only, W8A8): the model above.
// Smaller M, and bf16 W-only, by the number t256 of 256 x 128 blocks the
// output takes: the block shape whose grid splits most evenly over the 256
// CUs, and grids too small for two workgroups per CU split K over 4 wave
// groups inside the workgroup.  bf16 W-only keeps 64 x 128 wave tiles on the
// largest grids (half the conversion work per MFMA).
int pick_gemm_dl(bool i8, int xt, int64_t M, int64_t Nt, int64_t Kc) {
  if (M > 128 && i8) return model_pick(kPickI8, M, Nt, Kc);
  if (M > 128 && xt == XT_F16) return model_pick(kPickF16, M, Nt, Kc);
  const int64_t t256 = ((Nt + 15) / 16) * ((M + 127) / 128);
  const int64_t t128x64 = ((Nt + 7) / 8) * ((M + 63) / 64);
  if (i8) {
    // two K tiles per stage except on 192 x 128 blocks (three one-tile stages)
    if (t256 >= 1024 || (t256 >= 448 && t256 < 704)) return 13;  // 256 x 256
    if (t256 >= 320) return 19;                                   // 192 x 128
    if (t256 >= 224) return 14;                                   // 128 x 128
    if (t256 >= 160) return 20;                                   // 192 x 64
    // 128 x 64 also from 64 blocks of 256 x 128 up while K is short (there
    // the 64 x 64 K-split grid ran slower); long K keeps the in-workgroup split
    if (t256 >= 80 || (t256 >= 64 && Kc <= 96)) return 15;       // 128 x 64
    // 64 x 64, K split over 4 wave groups, while its grid fits one round of two
    // workgroups per CU (else 128 x 64)
    return ((Nt + 3) / 4) * ((M + 63) / 64) <= 2 * kCUs ? 8 : 15;
  }
  if (xt == XT_F16) {
    if (t256 >= 448 || (t256 >= 224 && t256 < 320)) return 0;  // 256 x 128
    if (t256 >= 320) return 18;                                 // 192 x 128
    if (t256 >= 160) return 16;                                 // 192 x 64
    if (t256 >= 112) return 3;                                  // 128 x 64
    // K split over 4 wave groups (one workgroup per CU): 192 x 64 (t256 >= 80),
    // 128 x 64 (>= 40) or 64 x 64 blocks.  When that grid needs a second round
    // of the 256 CUs, the largest of the three grids that fits one round runs,
    // else 128 x 64 blocks without the split (a second round nearly doubled
    // the time)
    const int64_t rb = (M + 63) / 64;
    const int64_t g8 = ((Nt + 3) / 4) * rb, g5 = ((Nt + 7) / 8) * rb, g17 = ((Nt + 11) / 12) * rb;
    const int id = t256 >= 80 ? 17 : (t256 >= 40 ? 5 : 8);
    if ((id == 17 ? g17 : (id == 5 ? g5 : g8)) <= kCUs) return id;
    if (g8 <= kCUs) return 8;
    if (g5 <= kCUs) return 5;
    if (g17 <= kCUs) return 17;
    return 3;
  }
  if (t256 >= 1536) return 10;
  if (t256 >= 256 || t128x64 >= 512) return 0;
  if (t128x64 >= 128) return 5;
  return 8;
}

// Mid-sized M (M <= 128): 64 x 64 blocks (configuration 22: one 16-row weight
// tile per wave, every token of the block in each wave, a 3-stage ring), with
// K split over S workgroups when the grid of B blocks leaves CUs idle:
// S = min(4, budget / B), budget 288 blocks for W8A8 and 768 for fp16 W-only
// (whose blocks carry twice the activation bytes per K tile and gain from more
// workgroups), each split keeping at least 4 stage steps.  Grids of more than
// 512 blocks keep the picker's configuration.  Measured on MI355X (the GEMM
// alone, weights rotating beyond the Infinity Cache, against the previous
// plan: 128 x 64 blocks split when fewer than 192 of them): W8A8 M = 128,
// N = 4096: 14.4 -> 11.8 us; N = 12288: 23.9 -> 21.0 us; N = 2560, K = 9728:
// 22.0 -> 16.2 us; fp16 W-only M = 128, N = 4096: 17.4 -> 13.2 us; N = 12288:
// 30.4 -> 25.6 us.  Only for operands that need no in-loop row sums: W8A8, and
// fp16 W-only with precomputed row sums (the staged fp32 / bf16 activations
// included).
constexpr int kMidId = 22;

DlPlan plan_gemm_dl(bool i8, int xt, int64_t M, int64_t Nt, int64_t Kc, bool rsp) {
  DlPlan p{pick_gemm_dl(i8, xt, M, Nt, Kc), 1, 0, 0};
  if (!i8 && !(xt == XT_F16 && rsp)) return p;
  if (M > 128) return p;
  const int64_t tiles = ((Nt + 3) / 4) * ((M + 63) / 64);
  if (tiles > 512) return p;
  p.id = kMidId;
  const int64_t steps = i8 && Kc % 2 == 0 ? Kc / 2 : Kc;  // stage steps of the configuration
  int64_t S = (i8 ? 288 : 768) / tiles;
  S = S < 1 ? 1 : (S > kMaxSplits ? kMaxSplits : S);
  while (S > 1 && steps / S < 4) --S;
  if (S == 1) return p;
  p.splits = (int)S;
  p.tiles = tiles;
  p.part_bytes = tiles * S * 64 * 64 * 4;  // one fp32 / int32 partial tile per split
  return p;
}

// Bytes of the split-K area (tile counters, then partial tiles) of a plan.
int64_t split_area_bytes(const DlPlan& p) {
  return p.splits > 1 ? ((p.tiles * 4 + 255) & ~(int64_t)255) + p.part_bytes : 0;
}

// Attach the split-K area to the GEMM arguments when the caller's scratch
// holds it; returns the counters the pre-pass must zero (null: no split).
static uint32_t* attach_split(GemmArgs& a, const DlPlan& p, uint8_t* area, int64_t area_bytes, int* ncount) {
  *ncount = 0;
  if (p.splits <= 1 || !area || area_bytes < split_area_bytes(p)) return nullptr;
  a.tcount = (uint32_t*)area;
  a.part = area + ((p.tiles * 4 + 255) & ~(int64_t)255);
  a.splits = p.splits;
  *ncount = (int)p.tiles;
  return a.tcount;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
constexpr int kBN = 128, kBM = 128, kWN = 2, kWM = 2;

W8Ws w8_ws_layout(int64_t M, int64_t K, int xt) {
  auto r256 = [](int64_t b) { return (b + 255) & ~(int64_t)255; };
  const int np = xt == XT_F32 || xt == XT_BF16 ? 1 : 0;  // one staged fp16 plane
  W8Ws l;
  l.rowsum = 0;
  l.rscale = r256(M * 4);
  l.planes = l.rscale + r256(M * 4);
  l.bytes = l.planes + r256(M * np * K * 2);
  return l;
}

// flags bit 8 of the direct-to-LDS GEMM: y and its row stride are 16-byte
// aligned (whole 16-byte output chunks from the LDS-staged epilogue).
inline int y16_flag(const void* y, int yt, int64_t ldy) {
  const int64_t es = yt == XT_F32 ? 4 : 2;
  return ((uintptr_t)y % 16 == 0 && (ldy * es) % 16 == 0) ? 8 : 0;
}

int launch_gemm_w8(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec, const uint8_t* packed,
                   const float* scale, const float* bias, int64_t N, void* y, int yt, int64_t ldy, void* ws,
                   int64_t ws_bytes, hipStream_t st, bool yvec) {
  const int64_t Nt = (N + 15) / 16, Kc = (K + 63) / 64;
  const int flags = (xvec ? 1 : 0) | (yvec ? 2 : 0) | y16_flag(y, yt, ldy);
  // the direct-to-LDS path addresses a block's rows and tiles with 32-bit offsets
  const bool dl = xvec && K % 64 == 0 && ldx <= ((int64_t)1 << 21) && K <= ((int64_t)1 << 21);
  const W8Ws l = w8_ws_layout(M, K, xt);
  const bool staged = dl && ws && ws_bytes >= l.bytes;
  if (dl && (xt != XT_F32 || staged)) {
    GemmArgs a{};
    a.x = x; a.ldx = ldx; a.M = (int)M; a.Kc = (int)Kc;
    a.packed = packed; a.scale = scale; a.bias = bias;
    a.N = (int)N; a.Nt = (int)Nt; a.y = y; a.yt = yt; a.ldy = ldy; a.flags = flags;
    const int gxt = staged ? XT_F16 : xt;  // fp32 / bf16 activations are staged as an fp16 plane
    // split K when the grid is small and the scratch after the layout holds the partials
    const DlPlan plan = plan_gemm_dl(false, gxt, M, Nt, Kc, staged);
    int ncount = 0;
    uint32_t* zero = staged ? attach_split(a, plan, (uint8_t*)ws + l.bytes, ws_bytes - l.bytes, &ncount) : nullptr;
    const int id = zero || plan.splits == 1 ? plan.id : pick_gemm_dl(false, gxt, M, Nt, Kc);
    if (staged) {
      uint8_t* w = (uint8_t*)ws;
      float* rowsum = (float*)(w + l.rowsum);
      a.rsum = rowsum;
      if (xt == XT_F16 && !zero && (id == 3 || id == 5 || id == 16)) {
        // fp16 x, no split: these three configurations sum the rows in their
        // K loop for less than the row-sum launch costs (measured over
        // M = 192 ... 1024, N = 2048 ... 24576, K = 2560 ... 12288: 128 x 64
        // blocks with K over 4 wave groups 6-7% faster, 128 x 64 and 192 x 64
        // blocks 0-4%; the larger blocks and the 64 x 64 split ran 2-30% slower
        // that way, and keep the pre-pass)
        a.rsum = nullptr;
      } else if (xt == XT_F16) {
        const int rc = launch_rowsum_f16(x, ldx, M, K, rowsum, st, zero, ncount);
        if (rc) return rc;
      } else {
        // fp32 / bf16: one scaled fp16 plane per row, then the fp16 GEMM
        _Float16* plane = (_Float16*)(w + l.planes);
        float* rscale = (float*)(w + l.rscale);
        const int rc = launch_stage_act(x, xt, ldx, M, K, plane, rowsum, rscale, st, zero, ncount);
        if (rc) return rc;
        a.x = plane; a.ldx = K; a.rscale = rscale;
        a.flags = flags | 1;
      }
    }
    return launch_gemm_dl_cfg(id, false, gxt, a, st);
  }
  dim3 grid((unsigned)((Nt + kBN / 16 - 1) / (kBN / 16)), (unsigned)((M + kBM - 1) / kBM)), block(kWN * kWM * 64);
  switch (xt) {
    case XT_F16: hipLaunchKernelGGL((gemm_w8_kernel<XT_F16, kBN, kBM, kWN, kWM>), grid, block, 0, st, x, ldx, (int)M, (int)K, (int)Kc, packed, scale, bias, (int)N, (int)Nt, y, yt, ldy, flags); break;
    case XT_BF16: hipLaunchKernelGGL((gemm_w8_kernel<XT_BF16, kBN, kBM, kWN, kWM>), grid, block, 0, st, x, ldx, (int)M, (int)K, (int)Kc, packed, scale, bias, (int)N, (int)Nt, y, yt, ldy, flags); break;
    case XT_F32: hipLaunchKernelGGL((gemm_w8_kernel<XT_F32, kBN, kBM, kWN, kWM>), grid, block, 0, st, x, ldx, (int)M, (int)K, (int)Kc, packed, scale, bias, (int)N, (int)Nt, y, yt, ldy, flags); break;
    default: return -2;
  }
  return check_launch();
}

int launch_gemm_w8a8(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec, const uint8_t* packed,
                     const float* scale, const int32_t* colsum, const float* bias, int64_t N, void* y, int yt,
                     int64_t ldy, int32_t* acc_out, float2* partials, int8_t* xq, float* qpbuf, hipStream_t st,
                     bool yvec, uint8_t* split, int64_t split_bytes) {
  const int64_t Nt = (N + 15) / 16, Kc = (K + 63) / 64, Kp = Kc * 64;
  if (Kp > ((int64_t)1 << 21)) return -1;  // 32-bit block offsets of the direct-to-LDS GEMM
  GemmArgs a{};
  const DlPlan plan = plan_gemm_dl(true, XT_F16, M, Nt, Kc, true);
  int ncount = 0;
  uint32_t* zero = attach_split(a, plan, split, split_bytes, &ncount);
  const int id = zero || plan.splits == 1 ? plan.id : pick_gemm_dl(true, XT_F16, M, Nt, Kc);
  const int nparts = minmax_nparts(M, K);
  const int prc = launch_minmax_partials(x, xt, M, K, ldx, partials, nparts, st, zero, ncount);
  if (prc) return prc;
  const int flags = (xvec ? 1 : 0) | (yvec ? 2 : 0) | y16_flag(y, yt, ldy);
  const int64_t chunks = M * (Kp / 16);
  // chunks per thread: 4 once that still gives >= 512 workgroups, 2 from 256
  // workgroups, else 1 (measured at K = 4096: M = 128 4.2 -> 3.1 us, M = 512
  // 4.4 -> 3.7 us, M = 2048 unchanged)
  const int qc = chunks >= (int64_t)256 * 4 * 512 ? 4 : (chunks >= (int64_t)256 * 2 * 256 ? 2 : 1);
  const dim3 qgrid((unsigned)((chunks + 256 * qc - 1) / (256 * qc)));
  const bool qvec = xvec && K % 16 == 0;
  const bool qdense = xvec && ldx == K && K % 64 == 0;  // flat rows in and out
#define SBQ_QUANT_DENSE1(XT_, QC_)                                                                                  \
  hipLaunchKernelGGL((quantize_dense_kernel<XT_, QC_>), qgrid, dim3(256), 0, st, x, chunks, partials, nparts, xq, qpbuf);
#define SBQ_QUANT_DENSE(XT_)                       \
  if (qc == 4) SBQ_QUANT_DENSE1(XT_, 4)            \
  else if (qc == 2) SBQ_QUANT_DENSE1(XT_, 2)       \
  else SBQ_QUANT_DENSE1(XT_, 1)
#define SBQ_QUANT_LAUNCH1(XT_, VEC_, QC_)                                                                          \
  hipLaunchKernelGGL((quantize_act_kernel<XT_, VEC_, QC_>), qgrid, dim3(256), 0, st, x, ldx, (int)M, (int)K, (int)Kp, \
                     partials, nparts, xq, qpbuf, flags);
#define SBQ_QUANT_LAUNCH(XT_)                       \
  if (qvec) {                                       \
    if (qc == 4) SBQ_QUANT_LAUNCH1(XT_, true, 4)    \
    else if (qc == 2) SBQ_QUANT_LAUNCH1(XT_, true, 2) \
    else SBQ_QUANT_LAUNCH1(XT_, true, 1)            \
  } else {                                          \
    if (qc == 4) SBQ_QUANT_LAUNCH1(XT_, false, 4)   \
    else if (qc == 2) SBQ_QUANT_LAUNCH1(XT_, false, 2) \
    else SBQ_QUANT_LAUNCH1(XT_, false, 1)           \
  }
  if (qdense) {
    switch (xt) {
      case XT_F16: SBQ_QUANT_DENSE(XT_F16) break;
      case XT_BF16: SBQ_QUANT_DENSE(XT_BF16) break;
      case XT_F32: SBQ_QUANT_DENSE(XT_F32) break;
      default: return -2;
    }
  } else {
    switch (xt) {
      case XT_F16: SBQ_QUANT_LAUNCH(XT_F16) break;
      case XT_BF16: SBQ_QUANT_LAUNCH(XT_BF16) break;
      case XT_F32: SBQ_QUANT_LAUNCH(XT_F32) break;
      default: return -2;
    }
  }
#undef SBQ_QUANT_DENSE
#undef SBQ_QUANT_DENSE1
#undef SBQ_QUANT_LAUNCH
#undef SBQ_QUANT_LAUNCH1
  int rc = check_launch();
  if (rc) return rc;
  // small M: the row-tile GEMV on the s8 rows where it beats the tiled GEMM
  // (the GEMM's plan is available when it needs no split area or has it)
  const bool alt = plan.splits == 1 || zero != nullptr;
  if (M > 16 && gemv_mt_applies(M, Kp, N, XT_S8, alt)) {
    GemvArgs g{};
    g.x = xq; g.ldx = Kp; g.M = (int)M; g.K = (int)Kp; g.Kc = (int)Kc;
    g.packed = packed; g.scale = scale; g.bias = bias; g.colsum = colsum;
    g.N = (int)N; g.Nt = (int)Nt; g.y = y; g.yt = yt; g.ldy = ldy; g.acc_out = acc_out; g.qpbuf = qpbuf;
    g.flags = kGemvXVec | (yvec ? kGemvYVec : 0);
    rc = launch_gemv_mt(g, XT_S8, st, alt);
    if (rc != -1) return rc;
  }
  a.x = xq; a.ldx = Kp; a.M = (int)M; a.Kc = (int)Kc;
  a.packed = packed; a.scale = scale; a.bias = bias; a.colsum = colsum;
  a.N = (int)N; a.Nt = (int)Nt; a.y = y; a.yt = yt; a.ldy = ldy; a.acc_out = acc_out; a.qpbuf = qpbuf;
  a.flags = flags;
  return launch_gemm_dl_cfg(id, true, XT_F16, a, st);
}

// Per-token symmetric W8A8: xq [M, Kp] s8 and s_t [M] from the row quantizer,
// then the fast GEMV (M <= 16) or the i8 GEMM with the per-token epilogue.
int launch_gemm_w8a8_token(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec,
                           const uint8_t* packed, const float* scale, const float* bias, int64_t N, void* y, int yt,
                           int64_t ldy, int32_t* acc_out, int8_t* xq, float* s_t, hipStream_t st, bool yvec) {
  const int64_t Nt = (N + 15) / 16, Kc = (K + 63) / 64, Kp = Kc * 64;
  if (Kp > ((int64_t)1 << 21)) return -1;  // 32-bit block offsets of the direct-to-LDS GEMM
  if (M <= 16 && xvec && K % 64 == 0) {
    // decode sizes with x of at most 8 chunks of 16 bytes per thread: one
    // launch, the GEMV quantizing each row itself (the row quantizer's
    // values, bit for bit); xq and s_t are not written
    GemvArgs g{};
    g.x = x; g.ldx = ldx; g.M = (int)M; g.K = (int)K; g.Kc = (int)Kc;
    g.packed = packed; g.scale = scale; g.bias = bias;
    g.N = (int)N; g.Nt = (int)Nt; g.y = y; g.yt = yt; g.ldy = ldy; g.acc_out = acc_out;
    g.flags = kGemvXVec | (yvec ? kGemvYVec : 0) | kGemvPerToken;
    int id = 0, ks = 0;
    if (pick_gemv_fast(M, K, N, xt, true, true, &id, &ks)) {
      const int frc = launch_gemv_fast_cfg(id, ks, g, xt, true, st);
      if (frc != -1) return frc;
    }
  }
  int rc = launch_quantize_rows_sym(x, xt, ldx, xvec, M, K, Kp, xq, s_t, st);
  if (rc) return rc;
  if (M <= 16) {  // decode sizes: the HBM-streaming GEMV on the s8 rows
    GemvArgs g{};
    g.x = xq; g.ldx = Kp; g.M = (int)M; g.K = (int)Kp; g.Kc = (int)Kc;
    g.packed = packed; g.scale = scale; g.bias = bias;
    g.N = (int)N; g.Nt = (int)Nt; g.y = y; g.yt = yt; g.ldy = ldy; g.acc_out = acc_out; g.rscale = s_t;
    g.flags = 1 | (yvec ? 2 : 0);
    int id = 0, ks = 0;
    if (pick_gemv_fast(M, Kp, N, XT_F16, false, true, &id, &ks)) {
      rc = launch_gemv_fast_cfg(id, ks, g, XT_S8, true, st);
      // s8 rows load their fragments directly: an x-in-LDS pick (id 0)
      // runs as its direct-fragment equivalent (id 3, D = 8, G = 1)
      if (rc == -1 && id == 0) rc = launch_gemv_fast_cfg(3, ks, g, XT_S8, true, st);
      if (rc != -1) return rc;
    }
  }
  GemmArgs a{};
  a.x = xq; a.ldx = Kp; a.M = (int)M; a.Kc = (int)Kc;
  a.packed = packed; a.scale = scale; a.bias = bias;
  a.N = (int)N; a.Nt = (int)Nt; a.y = y; a.yt = yt; a.ldy = ldy; a.acc_out = acc_out; a.rscale = s_t;
  a.flags = (yvec ? 2 : 0) | 4 | y16_flag(y, yt, ldy);
  return launch_gemm_dl_cfg(pick_gemm_dl(true, XT_F16, M, Nt, Kc), true, XT_F16, a, st);
}

}  // namespace sbq

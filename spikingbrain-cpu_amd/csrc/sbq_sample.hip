// sbq_sample.hip - the engine's sampling step on the GPU: temperature,
// top-k, top-p and the draw over the lm_head logits
// (spikingbrain_cpu/engine.py:29-42, paths relative to the reference
// repository), so that a non-greedy decode step leaves the logits on the GPU.
//
// Per row of fp32 logits x [V] (engine.py:29-42):
//   z = x / T                                 (IEEE fp32 division)
//   top_k > 0: kth = the k-th largest z (k = min(top_k, V)); z < kth is masked
//   p = softmax(z) = exp(z - max) / sum       (fp32)
//   0 < top_p < 1: a token is kept when the probability mass of the tokens
//   above it is below top_p (the reference's sorted `cumsum - p < top_p`)
//   token = the first index i (vocabulary order) whose prefix mass of kept
//   tokens exceeds u * (kept mass), u in [0, 1) supplied by the caller (the
//   inverse of the distribution torch.multinomial draws from).
//
// No sort: the k-th largest z and the top-p boundary are found by radix
// selection over an order-preserving 32-bit key of z, 8 bits per pass, from
// histograms of token counts (top-k) or of the mass exp(z - max) (top-p), in
// 2^-40 fixed point, so that every sum is exact and independent of the order
// the atomics land in; top_p is applied to the kept mass as top_p * sum,
// which is the normalized condition.  Each workgroup builds its histogram in
// LDS and adds it into the pass's row histogram with device-scope atomics
// (the first launch zeroes those; top-k's first pass, in that launch, keeps
// one histogram per workgroup instead).  Every launch reads the row again
// from L2 (608 KB at V = 151936); a workgroup that needs the outcome of the
// previous pass re-derives it from that pass's histogram (identical in every
// workgroup), so no workgroup waits for another.  The first pass of each
// selection rides on the launch before it (the max pass, the softmax-sum
// pass).  Rows are independent (grid.y).  Differences from
// the reference's sort-based form: the top-p rule walks the tokens in the
// order of z, where the sort walks the fp32 probabilities, so of two tokens
// whose probabilities round to the same fp32 value the larger z comes first
// (the sort leaves the order of equal values open); and a token's mass is
// exp(z - max) truncated to 2^-40.  Tokens whose z ties at the top-p boundary
// are kept as the sort keeps them: as many as its rule admits, the first ones
// in vocabulary order (the order a stable sort gives them).
#include <stdint.h>

#include "sbq_common.h"
#include "sbq_launch.h"

namespace sbq {

constexpr int kSampThreads = 1024;
constexpr int kSampMaxBlocks = 64;   // workgroups per row (one wave's lanes sum their per-workgroup values)
constexpr int kSampCopies = 16;      // LDS copies of each histogram bin (atomics of one wave spread over them)
constexpr double kSampFix = 1099511627776.0;  // 2^40: exp(z - max) in (0, 1] -> fixed point

// Per-row scratch, from the row's first byte (each part 256-byte aligned).
struct SampRow {
  static constexpr int64_t kHead = 0;                       // SampHead
  static constexpr int64_t kMax = 256;                      // float [G]
  static constexpr int64_t kNan = kMax + 512;               // int [G]
  static constexpr int64_t kEsum = kNan + 512;              // uint64 [G]: mass of the tokens top-k keeps
  static constexpr int64_t kBsum = kEsum + 512;             // uint64 [G]: mass of the tokens both keep (boundary ties aside)
  static constexpr int64_t kTie = kBsum + 512;              // int [G]: tokens of the top-p boundary key
  static constexpr int64_t kState = kTie + 256;             // SampState [2]
  static constexpr int64_t kHist = kState + 256;            // uint64 [G][256]: top-k pass 0, per workgroup
  static constexpr int64_t kGh = kHist + kSampMaxBlocks * 256 * 8;  // uint64 [7][256]: the later passes' sums
  static constexpr int64_t kBytes = kGh + 7 * 256 * 8;
};
static_assert(kSampMaxBlocks * 8 <= 512 && kSampMaxBlocks * 4 <= 256 && kSampMaxBlocks <= 64,
              "per-block arrays fit their slots and one wave");

struct SampHead {
  uint32_t kth;    // key of the k-th largest z (0: no top-k)
  uint32_t tkey;   // key of the top-p boundary (0: no top-p)
  float m;         // max z
  int valid;       // 0: a NaN or an infinite max (the reference raises)
  int tie_n;       // top-p keeps the first tie_n tokens of key tkey (vocabulary order) ...
  int pad;
  uint64_t tie_f;  // ... each of mass tie_f (0: no such tokens)
};

// Radix descent state before a pass: the key bits found so far and the
// remaining rank (top-k) or the mass above the region (top-p).
struct SampState {
  uint32_t prefix;
  uint32_t pad;
  uint64_t rest;
};

struct SampArgs {
  const float* x;
  int64_t ld;
  int V, G, per;
  float T;
  int k;                 // min(top_k, V), or 0
  double top_p;          // 0 without top-p
  uint8_t* ws;
  int64_t ws_row;        // bytes per row (SampRow::kBytes)
  const float* u;        // [M] uniforms in [0, 1)
  int64_t* tokens;       // [M]
};

// Order-preserving key: a < b as floats <=> key(a) < key(b); -0 as +0.
__device__ __forceinline__ uint32_t samp_key(float z) {
  const uint32_t b = __float_as_uint(z == 0.0f ? 0.0f : z);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// z of a key (the inverse of samp_key; +0 for the key of zeros)
__device__ __forceinline__ float samp_unkey(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ float samp_z(const SampArgs& a, const float* row, int i) { return row[i] / a.T; }

// fixed-point mass exp(z - m) of a token top-k keeps (0 for masked ones)
__device__ __forceinline__ uint64_t samp_efix(float z, uint32_t kth, float m) {
  if (samp_key(z) < kth) return 0;
  return (uint64_t)((double)expf(z - m) * kSampFix);  // exp(z - m) <= 1: exact in double after the scaling
}

// The top-p bound on the mass above a token: mass_above < top_p * S (S: the
// mass top-k keeps) <=> mass_above < thr, for integer masses.
__device__ __forceinline__ uint64_t samp_thr(double top_p, uint64_t S) { return (uint64_t)ceil(top_p * (double)S); }

__device__ __forceinline__ uint8_t* samp_row_ws(const SampArgs& a) { return a.ws + (int64_t)blockIdx.y * a.ws_row; }

// LDS histogram of 256 bins x kSampCopies (lane l adds to copy l % copies,
// so a wave whose keys share a bin hits kSampCopies addresses, not one).
__device__ __forceinline__ void hist_clear(uint64_t* H) {
  for (int b = threadIdx.x; b < 256 * kSampCopies; b += blockDim.x) H[b] = 0;
}
__device__ __forceinline__ void hist_add(uint64_t* H, uint32_t bin, uint64_t v) {
  atomicAdd((unsigned long long*)&H[bin * kSampCopies + (threadIdx.x & (kSampCopies - 1))], (unsigned long long)v);
}
__device__ __forceinline__ void hist_store(const uint64_t* H, uint64_t* out) {
  for (int b = threadIdx.x; b < 256; b += blockDim.x) {
    uint64_t s = 0;
#pragma unroll
    for (int c = 0; c < kSampCopies; ++c) s += H[b * kSampCopies + c];
    out[b] = s;
  }
}
// add the workgroup's histogram into the row's (zeroed by the first launch)
__device__ __forceinline__ void hist_accumulate(const uint64_t* H, uint64_t* gh) {
  for (int b = threadIdx.x; b < 256; b += blockDim.x) {
    uint64_t s = 0;
#pragma unroll
    for (int c = 0; c < kSampCopies; ++c) s += H[b * kSampCopies + c];
    if (s) __hip_atomic_fetch_add((unsigned long long*)&gh[b], (unsigned long long)s, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
  }
}

__device__ __forceinline__ uint64_t samp_block_sum_u64(uint64_t v, uint64_t* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  uint64_t s = 0;
  for (int i = 0; i < nw; ++i) s += red[i];
  __syncthreads();
  return s;
}

// Two block sums at once (one pair of barriers); red: 32 words.
__device__ __forceinline__ void samp_block_sum2_u64(uint64_t& v0, uint64_t& v1, uint64_t* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    v0 += __shfl_xor(v0, o);
    v1 += __shfl_xor(v1, o);
  }
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[w] = v0;
    red[16 + w] = v1;
  }
  __syncthreads();
  uint64_t s0 = 0, s1 = 0;
  for (int i = 0; i < nw; ++i) {
    s0 += red[i];
    s1 += red[16 + i];
  }
  __syncthreads();
  v0 = s0;
  v1 = s1;
}

// Sum of v over the G <= 64 lanes of one wave (exact), every lane the result.
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// sum over g < G of a per-workgroup array, by the lanes of each wave (one
// load per lane, all in flight; identical in every wave and workgroup)
__device__ __forceinline__ uint64_t samp_sum_g(const uint64_t* p, int G) {
  const int lane = threadIdx.x & 63;
  return wave_sum_u64(lane < G ? p[lane] : 0);
}

// One radix step from the previous pass's histograms (every workgroup of the
// row computes the same result): top-k (MASS false) takes the digit whose
// bin holds the remaining rank counted from the top; top-p (MASS true) the
// lowest digit whose bins above leave the mass above the region below thr.
// The G histograms are summed by all threads (four partial sums per bin,
// added in a fixed order); wave 0 then finds the digit, four bins per lane,
// with suffix sums across the lanes.  P: 4 x 256 words of LDS.
template <bool MASS>
__device__ SampState samp_descend(const uint64_t* hist, int G, SampState st, uint64_t thr, uint64_t* P,
                                  SampState* out) {
  const int t = threadIdx.x, bin = t & 255, part = t >> 8;  // blockDim.x == 1024: parts 0..3
  uint64_t s = 0;
  for (int g = part; g < G; g += 4) s += hist[g * 256 + bin];
  P[part * 256 + bin] = s;
  if (t == 0) {  // the result if no bin qualifies (an empty or invalid row): the top bin
    SampState r = st;
    r.prefix = (st.prefix << 8) | 255u;
    *out = r;
  }
  __syncthreads();
  if (t < 64) {
    const int lane = t;
    uint64_t h[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int b = 4 * lane + j;
      h[j] = P[b] + P[256 + b] + P[512 + b] + P[768 + b];
    }
    const uint64_t local = h[0] + h[1] + h[2] + h[3];
    uint64_t suf = local;  // sum over lanes >= lane
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t v = __shfl_down(suf, o);
      if (lane + o < 64) suf += v;
    }
    const uint64_t above_lane = suf - local;  // bins of higher lanes
    // cum[j]: mass or count of the bins above bin 4 * lane + j
    const uint64_t cum3 = above_lane, cum2 = cum3 + h[3], cum1 = cum2 + h[2], cum0 = cum1 + h[1];
    const uint64_t cum[4] = {cum0, cum1, cum2, cum3};
    if constexpr (!MASS) {
      // the crossing bin: cum < rest <= cum + h (exactly one bin of the wave)
#pragma unroll
      for (int j = 3; j >= 0; --j)
        if (cum[j] < st.rest && st.rest <= cum[j] + h[j]) {
          SampState r = st;
          r.rest -= cum[j];
          r.prefix = (st.prefix << 8) | (uint32_t)(4 * lane + j);
          *out = r;
        }
    } else {
      // qualifying bins (rest + cum < thr) are those from some b0 up; the
      // lowest lane holding one holds b0
      int lowj = -1;
#pragma unroll
      for (int j = 3; j >= 0; --j)
        if (st.rest + cum[j] < thr) lowj = j;
      const uint64_t any = __ballot(lowj >= 0);
      const int lead = any ? __ffsll((long long)any) - 1 : -1;
      if (lane == lead) {
        SampState r = st;
        r.rest += cum[lowj];
        r.prefix = (st.prefix << 8) | (uint32_t)(4 * lane + lowj);
        *out = r;
      }
    }
  }
  __syncthreads();
  const SampState r = *out;
  __syncthreads();
  return r;
}

// First launch: max of z and NaN count per workgroup; with top-k, pass 0 of
// its selection (counts by the key's top byte).
__global__ __launch_bounds__(kSampThreads) void samp_first_kernel(SampArgs a) {
  __shared__ uint64_t H[256 * kSampCopies];
  __shared__ float mred[16];
  __shared__ int nred[16];
  const float* row = a.x + (int64_t)blockIdx.y * a.ld;
  uint8_t* w = samp_row_ws(a);
  const bool topk = a.k > 0;
  if (topk) hist_clear(H);
  if (blockIdx.x == 0)  // the row histograms of the later passes
    for (int b = threadIdx.x; b < 7 * 256; b += blockDim.x) ((uint64_t*)(w + SampRow::kGh))[b] = 0;
  __syncthreads();
  const int i0 = blockIdx.x * a.per, i1 = min(i0 + a.per, a.V);
  float mx = -INFINITY;
  int nan = 0;
  for (int i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
    const float z = samp_z(a, row, i);
    nan += z != z;
    mx = fmaxf(mx, z);
    if (topk) hist_add(H, samp_key(z) >> 24, 1);
  }
  mx = wave_max(mx);
  nan = wave_sum_i(nan);
  const int wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    mred[wv] = mx;
    nred[wv] = nan;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float m = mred[0];
    int n = nred[0];
    for (int i = 1; i < nw; ++i) {
      m = fmaxf(m, mred[i]);
      n += nred[i];
    }
    ((float*)(w + SampRow::kMax))[blockIdx.x] = m;
    ((int*)(w + SampRow::kNan))[blockIdx.x] = n;
    if (topk && blockIdx.x == 0) ((SampState*)(w + SampRow::kState))[0] = SampState{0u, 0u, (uint64_t)a.k};
  }
  if (topk) hist_store(H, (uint64_t*)(w + SampRow::kHist) + blockIdx.x * 256);
}

// Radix pass `pass` (1..3) of the top-k selection (MASS false: token counts)
// or of the top-p boundary (MASS true: fixed-point mass of the tokens top-k
// keeps).  Row histograms: top-k pass p in gh[p - 1] (its pass 0: the
// per-workgroup histograms), top-p pass p in gh[3 + p]; the descent state
// alternates between st[0] and st[1].
template <bool MASS>
__global__ __launch_bounds__(kSampThreads) void samp_select_kernel(SampArgs a, int pass) {
  __shared__ uint64_t H[256 * kSampCopies];
  __shared__ SampState bcast;
  const float* row = a.x + (int64_t)blockIdx.y * a.ld;
  uint8_t* w = samp_row_ws(a);
  uint64_t* gh = (uint64_t*)(w + SampRow::kGh);
  SampState* st = (SampState*)(w + SampRow::kState);
  uint32_t kth = 0;
  float m = 0.0f;
  uint64_t thr = 0;
  if constexpr (MASS) {
    const SampHead* h = (const SampHead*)(w + SampRow::kHead);
    kth = h->kth;
    m = h->m;
    thr = samp_thr(a.top_p, samp_sum_g((const uint64_t*)(w + SampRow::kEsum), a.G));
  }
  const uint64_t* src = MASS ? gh + (3 + pass - 1) * 256
                             : (pass == 1 ? (const uint64_t*)(w + SampRow::kHist) : gh + (pass - 2) * 256);
  const int srcG = !MASS && pass == 1 ? a.G : 1;
  const SampState cur = samp_descend<MASS>(src, srcG, st[(pass - 1) & 1], thr, H, &bcast);
  hist_clear(H);
  __syncthreads();
  const int i0 = blockIdx.x * a.per, i1 = min(i0 + a.per, a.V);
  const int hi = 32 - 8 * pass, lo = 24 - 8 * pass;
  for (int i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
    const float z = samp_z(a, row, i);
    const uint32_t key = samp_key(z);
    if ((key >> hi) != cur.prefix) continue;
    const uint32_t bin = (key >> lo) & 255u;
    if constexpr (MASS) {
      const uint64_t f = samp_efix(z, kth, m);
      if (f) hist_add(H, bin, f);
    } else {
      hist_add(H, bin, 1);
    }
  }
  __syncthreads();
  hist_accumulate(H, gh + (MASS ? 3 + pass : pass - 1) * 256);
  if (blockIdx.x == 0 && threadIdx.x == 0) st[pass & 1] = cur;
}

// Softmax mass over the tokens top-k keeps, per workgroup (after the top-k
// passes: its last digit is derived here); with top-p, pass 0 of its
// selection.  Workgroup 0 records the k-th largest key, the max and validity.
__global__ __launch_bounds__(kSampThreads) void samp_soft_kernel(SampArgs a) {
  __shared__ uint64_t H[256 * kSampCopies];
  __shared__ SampState bcast;
  __shared__ uint64_t red[16];
  const float* row = a.x + (int64_t)blockIdx.y * a.ld;
  uint8_t* w = samp_row_ws(a);
  uint32_t kth = 0;
  if (a.k > 0)
    kth = samp_descend<false>((const uint64_t*)(w + SampRow::kGh) + 2 * 256, 1,
                              ((const SampState*)(w + SampRow::kState))[1], 0, H, &bcast)
              .prefix;
  const float* maxp = (const float*)(w + SampRow::kMax);
  const int* nanp = (const int*)(w + SampRow::kNan);
  const int lane = threadIdx.x & 63;
  const float m = wave_max(lane < a.G ? maxp[lane] : -INFINITY);
  const int nan = wave_sum_i(lane < a.G ? nanp[lane] : 0);
  const bool valid = nan == 0 && m < INFINITY && m > -INFINITY;
  const bool topp = a.top_p > 0.0;
  if (topp) hist_clear(H);
  __syncthreads();
  const int i0 = blockIdx.x * a.per, i1 = min(i0 + a.per, a.V);
  uint64_t part = 0;
  if (valid)
    for (int i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
      const float z = samp_z(a, row, i);
      const uint64_t f = samp_efix(z, kth, m);
      part += f;
      if (topp && f) hist_add(H, samp_key(z) >> 24, f);
    }
  const uint64_t s = samp_block_sum_u64(part, red);  // its barriers also end the histogram adds
  if (threadIdx.x == 0) {
    ((uint64_t*)(w + SampRow::kEsum))[blockIdx.x] = s;
    if (blockIdx.x == 0) {
      SampHead* h = (SampHead*)(w + SampRow::kHead);
      h->kth = kth;
      h->tkey = 0;
      h->m = m;
      h->valid = valid ? 1 : 0;
      h->tie_n = 0;
      h->tie_f = 0;
      if (topp) ((SampState*)(w + SampRow::kState))[0] = SampState{0u, 0u, 0u};
    }
  }
  if (topp) hist_accumulate(H, (uint64_t*)(w + SampRow::kGh) + 3 * 256);
}

// With top-p: the mass of the tokens both cuts keep, per workgroup (the top-p
// boundary's last digit is derived here); workgroup 0 records the boundary.
// The tokens of the boundary key share one z, so one mass f.  The reference's
// sort puts them together (in vocabulary order: a stable sort) and its rule
// keeps the j-th of them while the mass above it, A + j f, stays below
// top_p: the first n = ceil((thr - A) / f) of them (A: the mass of the keys
// above, the descent's rest).  When n is below their count, they are counted
// per workgroup here and left out of its mass, and the draw adds f for each
// of the first n; otherwise all of them are kept, as every key above.
__global__ __launch_bounds__(kSampThreads) void samp_bsum_kernel(SampArgs a) {
  __shared__ uint64_t H[1024];
  __shared__ SampState bcast;
  __shared__ uint64_t red[32];
  const float* row = a.x + (int64_t)blockIdx.y * a.ld;
  uint8_t* w = samp_row_ws(a);
  SampHead* h = (SampHead*)(w + SampRow::kHead);
  const uint64_t S = samp_sum_g((const uint64_t*)(w + SampRow::kEsum), a.G);
  const uint64_t thr = samp_thr(a.top_p, S);
  const uint64_t* last = (const uint64_t*)(w + SampRow::kGh) + 6 * 256;  // pass 3: masses by the key's low byte
  const SampState fin = samp_descend<true>(last, 1, ((const SampState*)(w + SampRow::kState))[1], thr, H, &bcast);
  const uint32_t tkey = fin.prefix;
  const uint32_t kth = h->kth;
  const float m = h->m;
  const bool valid = h->valid != 0;
  const uint32_t lim = kth > tkey ? kth : tkey;
  const int i0 = blockIdx.x * a.per, i1 = min(i0 + a.per, a.V);
  uint64_t part = 0, ties = 0;  // the mass of every kept key, the tokens of the boundary key
  if (valid)
    for (int i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
      const float z = samp_z(a, row, i);
      const uint32_t key = samp_key(z);
      ties += key == tkey;
      if (key >= lim) part += samp_efix(z, kth, m);
    }
  samp_block_sum2_u64(part, ties, red);
  if (threadIdx.x == 0) {
    // the boundary key's tokens: mass f0 each, tmass in all (0: none kept by
    // top-k), from the pass-3 histogram the descent left in LDS (four
    // partial sums per bin); the same decision in every workgroup
    const uint32_t tb = tkey & 255u;
    const uint64_t tmass = H[tb] + H[256 + tb] + H[512 + tb] + H[768 + tb];
    const uint64_t f0 = valid && tmass ? samp_efix(samp_unkey(tkey), kth, m) : 0;
    uint64_t n = 0, cnt = 0;
    // one token (tmass == f0, the usual case) is kept whole; the quotients
    // below are for a key of several tokens (thr > rest: the key qualifies)
    if (f0 && tmass > f0 && thr > fin.rest) {
      // cnt = tmass / f0 (every token of the key adds the same f0; an
      // integer <= V, so the rounded double quotient is exact) and n =
      // min(cnt, ceil(need / f0)): below tmass the quotient is < cnt, and
      // its double estimate is corrected by at most one either way
      cnt = (uint64_t)((double)tmass / (double)f0 + 0.5);
      const uint64_t need = thr - fin.rest;
      if (need >= tmass) {
        n = cnt;
      } else {
        n = (uint64_t)ceil((double)need / (double)f0);
        if (n > 0 && (n - 1) * f0 >= need) --n;
        if (n * f0 < need) ++n;
      }
    }
    // only a boundary key that keeps part of its tokens is split off (usually
    // it holds one token, which is kept): its tokens leave the slice's mass
    // (each added f0 to it) and are counted instead
    const uint64_t f = n < cnt ? f0 : 0;
    ((uint64_t*)(w + SampRow::kBsum))[blockIdx.x] = f ? part - ties * f0 : part;
    ((int*)(w + SampRow::kTie))[blockIdx.x] = f ? (int)ties : 0;
    if (blockIdx.x == 0) {
      h->tkey = tkey;
      h->tie_f = f;
      h->tie_n = (int)n;
    }
  }
}

// The draw: the first index whose prefix of kept mass exceeds u * total.
// One workgroup per row; thread t owns a contiguous run of the chosen
// workgroup slice; wave scans, then the wave totals in order.  With top-p,
// of the tokens of the boundary key only the first tie_n (vocabulary order)
// count, tie_f each: a slice keeps those of them that the slices before it
// leave, and a token's rank among them is the slice's start plus the ties
// of the threads before it and of its own run before it.
__global__ __launch_bounds__(kSampThreads) void samp_pick_kernel(SampArgs a, int use_bsum) {
  __shared__ uint64_t wtot[16];
  __shared__ int wtie[16];
  __shared__ int found;
  const int row_i = blockIdx.y;
  const float* row = a.x + (int64_t)row_i * a.ld;
  const uint8_t* w = samp_row_ws(a);
  const SampHead hd = *(const SampHead*)(w + SampRow::kHead);  // the whole head in one load
  if (!hd.valid) {
    if (threadIdx.x == 0) a.tokens[row_i] = -1;
    return;
  }
  const uint64_t* bsum = (const uint64_t*)(w + (use_bsum ? SampRow::kBsum : SampRow::kEsum));
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint64_t tf = use_bsum ? hd.tie_f : 0;
  const int tn = use_bsum ? hd.tie_n : 0;
  // every wave, when the boundary key is split off (tf: uniform, the row's
  // head): the boundary ties of the slices in lanes and their prefix ...
  int tbefore_g = 0, tkeep_g = 0;  // ties in the slices before, ties the slice keeps
  if (tf) {
    const int tc_g = lane < a.G ? ((const int*)(w + SampRow::kTie))[lane] : 0;
    int tpre_g = tc_g;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(tpre_g, o);
      if (lane >= o) tpre_g += v;
    }
    tbefore_g = tpre_g - tc_g;
    tkeep_g = min(max(tn - tbefore_g, 0), tc_g);
  }
  // ... the slice masses, their inclusive prefix, the total
  const uint64_t mine_g = lane < a.G ? bsum[lane] + tf * (uint64_t)tkeep_g : 0;
  uint64_t pre_g = mine_g;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t v = __shfl_up(pre_g, o);
    if (lane >= o) pre_g += v;
  }
  const uint64_t total = __shfl(pre_g, 63);
  double uf = (double)a.u[row_i];
  uf = uf < 0.0 ? 0.0 : uf;
  uint64_t target = (uint64_t)(uf * (double)total);
  if (target >= total) target = total - 1;  // u = 1 (outside [0, 1)) takes the last kept token
  // the slice whose prefix first exceeds the target (the last slice at the latest)
  const uint64_t over = __ballot(lane < a.G && pre_g > target);
  const int g = over ? __ffsll((long long)over) - 1 : a.G - 1;
  target -= __shfl(pre_g - mine_g, g);  // within workgroup slice g
  const int trank0 = __shfl(tbefore_g, g);
  const uint32_t kth = hd.kth, tkey = hd.tkey;
  const uint32_t lim = kth > tkey ? kth : tkey;
  const float m = hd.m;
  const int i0 = g * a.per, i1 = min(i0 + a.per, a.V);
  const int e = (i1 - i0 + (int)blockDim.x - 1) / (int)blockDim.x;  // elements per thread
  const int t0 = i0 + threadIdx.x * e, t1 = min(t0 + e, i1);
  // the kept mass of token i (rank: the boundary ties met so far)
  auto kept = [&](int i, int& rank) -> uint64_t {
    const float z = samp_z(a, row, i);
    const uint32_t key = samp_key(z);
    if (tf && key == tkey) return rank++ < tn ? tf : 0;
    return key >= lim ? samp_efix(z, kth, m) : 0;
  };
  // this thread's run: the mass of its other tokens and its boundary ties
  uint64_t mine = 0;
  int myt = 0;
  for (int i = t0; i < t1; ++i) {
    const float z = samp_z(a, row, i);
    const uint32_t key = samp_key(z);
    if (tf && key == tkey)
      ++myt;
    else if (key >= lim)
      mine += samp_efix(z, kth, m);
  }
  int rank0 = 0;  // rank of this run's first boundary tie
  if (tf) {  // uniform: the row's head
    int tincl = myt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(tincl, o);
      if (lane >= o) tincl += v;
    }
    if (lane == 63) wtie[wv] = tincl;
    __syncthreads();
    int tbase = trank0;
    for (int i = 0; i < wv; ++i) tbase += wtie[i];
    rank0 = tbase + tincl - myt;
    mine += tf * (uint64_t)min(max(tn - rank0, 0), myt);  // its ties below rank tn
  }
  // inclusive scan within the wave, then the wave totals in wave order
  uint64_t incl = mine;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t v = __shfl_up(incl, o);
    if (lane >= o) incl += v;
  }
  if (lane == 63) wtot[wv] = incl;
  if (threadIdx.x == 0) found = -1;
  __syncthreads();
  uint64_t base = 0;
  for (int i = 0; i < wv; ++i) base += wtot[i];
  incl += base;
  const uint64_t excl = incl - mine;
  if (excl <= target && target < incl) {
    uint64_t c = excl;
    int rank = rank0;
    for (int i = t0; i < t1; ++i) {
      c += kept(i, rank);
      if (c > target) {
        found = i;
        break;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) a.tokens[row_i] = found;
}

int64_t sample_workspace_bytes(int64_t M) { return M * SampRow::kBytes; }

int launch_sample_rows(const float* x, int64_t M, int64_t V, int64_t ld, float T, int64_t top_k, float top_p,
                       const float* u, int64_t* tokens, void* ws, hipStream_t st) {
  SampArgs a{};
  a.x = x;
  a.ld = ld;
  a.V = (int)V;
  a.G = (int)((V + 2047) / 2048);
  if (a.G > kSampMaxBlocks) a.G = kSampMaxBlocks;
  a.per = (int)((V + a.G - 1) / a.G);
  a.T = T;
  a.k = top_k > 0 && top_k < V ? (int)top_k : 0;
  a.top_p = top_p > 0.0f && top_p < 1.0f ? (double)top_p : 0.0;
  a.ws = (uint8_t*)ws;
  a.ws_row = SampRow::kBytes;
  a.u = u;
  a.tokens = tokens;
  const dim3 grid((unsigned)a.G, (unsigned)M), block(kSampThreads);
  hipLaunchKernelGGL(samp_first_kernel, grid, block, 0, st, a);
  if (a.k)
    for (int p = 1; p < 4; ++p) hipLaunchKernelGGL(samp_select_kernel<false>, grid, block, 0, st, a, p);
  hipLaunchKernelGGL(samp_soft_kernel, grid, block, 0, st, a);
  if (a.top_p > 0.0) {
    for (int p = 1; p < 4; ++p) hipLaunchKernelGGL(samp_select_kernel<true>, grid, block, 0, st, a, p);
    hipLaunchKernelGGL(samp_bsum_kernel, grid, block, 0, st, a);
  }
  hipLaunchKernelGGL(samp_pick_kernel, dim3(1, (unsigned)M), block, 0, st, a, a.top_p > 0.0 ? 1 : 0);
  return check_launch();
}

}  // namespace sbq

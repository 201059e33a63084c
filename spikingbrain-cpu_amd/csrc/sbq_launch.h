// sbq_launch.h - internal host-side launchers shared between the kernel files
// and the C ABI (sbq_abi.hip).  Return 0 or a negative SBQ_ERR_* code.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sbq {

inline int check_launch() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : -5;
}

int launch_quantize_per_channel(const void* w, int wt, int64_t N, int64_t K, int64_t ldw, int8_t* q,
                                int64_t ldq, float* scale, hipStream_t st);
int launch_repack(const int8_t* q, int64_t N, int64_t K, int64_t ldq, uint8_t* packed, int32_t* colsum,
                  hipStream_t st);
int launch_unpack(const uint8_t* packed, int64_t N, int64_t K, int8_t* q, int64_t ldq, hipStream_t st);

int minmax_nparts(int64_t M, int64_t K);
// zero / nzero (optional): counters the pre-pass zeroes for the split-K GEMM
// launched after it on the same stream.
int launch_minmax_partials(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, float2* partials,
                           int nparts, hipStream_t st, uint32_t* zero = nullptr, int nzero = 0);
int launch_qparams(const float2* partials, int nparts, float* scale_out, int32_t* zp_out, hipStream_t st);
int launch_argmax_rows(const float* y, int64_t M, int64_t N, int64_t ldy, int64_t* out, hipStream_t st);
// The engine's non-greedy sampling step (sbq_sample.hip) over rows of fp32
// logits; ws: sample_workspace_bytes(M), 256-byte aligned.  Vocabularies up
// to kSampMaxVocab: a row's fixed-point mass (each token at most 2^40) then
// stays below 2^63.
constexpr int64_t kSampMaxVocab = (int64_t)1 << 23;
int64_t sample_workspace_bytes(int64_t M);
int launch_sample_rows(const float* x, int64_t M, int64_t V, int64_t ld, float T, int64_t top_k, float top_p,
                       const float* u, int64_t* tokens, void* ws, hipStream_t st);

// True when the streaming GEMV kernels take this M and K (otherwise the GEMM).
bool gemv_supports(int64_t M, int64_t K, bool w8a8, int xt);
// The general GEMV's configuration for an [M, K] input (sbq_gemv_config):
// info[0..8] = ok, row tiles of x, weight tiles per group, K tiles per wave,
// waves, activation mode, staging chunks per thread, LDS bytes, and whether a
// kernel instance exists for it.
int gemv_config_info(int64_t M, int64_t K, bool w8a8, int xt, int32_t* info);

// Decode fast path (sbq_gemv_fast.hip): M <= 16, K % 64 == 0, aligned x rows.
// pick_gemv_fast chooses a configuration id and the waves per workgroup;
// launch_gemv_fast_cfg returns -1 when that configuration cannot run the shape.
struct GemvArgs;
struct GemvSeg;
bool pick_gemv_fast(int64_t M, int64_t K, int64_t N, int xt, bool w8a8, bool xvec, int* id, int* ks);
int launch_gemv_fast_cfg(int id, int ks, const GemvArgs& a, int xt, bool w8a8, hipStream_t st);
// Decode over several 16-row tiles of x (16 < M <= 64): weight-only on fp16 /
// bf16 x, or int8-dyn on pre-quantized s8 rows (xt XT_S8).  gemm_alt: the
// caller can run the tiled GEMM's mid-sized-M plan instead (then the path is
// taken on fewer shapes).
bool gemv_mt_applies(int64_t M, int64_t K, int64_t N, int xt, bool gemm_alt);
int launch_gemv_mt(const GemvArgs& a, int xt, hipStream_t st, bool gemm_alt);
int launch_gemv_w8_mt(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec, const uint8_t* packed,
                      const float* scale, const float* bias, int64_t N, void* y, int yt, int64_t ldy, hipStream_t st,
                      bool yvec, bool gemm_alt);
// Grouped launch: a.seg / a.nseg hold 2..kGemvMaxSeg linears (w8a8: int8-dyn
// with the activation min/max reduced in the kernel).
int launch_gemv_fast_grouped(int id, int ks, GemvArgs a, int xt, bool w8a8, hipStream_t st);
// n independent linears sharing M, K and dtypes in one launch (x / weight /
// scale / bias / colsum / y / strides / N / Nt per segment), weight-only or
// int8-dyn (w8a8); -1 when the fast path does not apply.
int launch_gemv_w8_grouped(const GemvSeg* segs, int n, int xt, int64_t M, int64_t K, bool xvec, int yt, bool yvec,
                           hipStream_t st, bool w8a8 = false);

// Fused greedy token of the decode GEMV (fp32 y, M <= 16): the argmax state
// (kArgmaxStateBytes, zero before a launch, zero again after it) and the
// int64 token per row.  The launcher sets `fused` when the GEMV it ran also
// picked the tokens; otherwise the caller picks them from y.
struct GemvArgmaxOut {
  uint8_t* state;
  int64_t* idx;
  bool fused;
};

// Weight-only linear.  xvec: x and every row of x start 16-byte aligned (vector
// loads allowed).  yvec: y rows are 16-byte aligned and N % 4 == 0.
int launch_gemv_w8(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec, const uint8_t* packed,
                   const float* scale, const float* bias, int64_t N, void* y, int yt, int64_t ldy, hipStream_t st,
                   bool yvec, GemvArgmaxOut* am = nullptr);
// ws: device scratch (nullable, 256-byte aligned) of ws_bytes bytes, laid out
// by w8_ws_layout.  With enough of it the fp16 GEMM takes its per-row sums of x
// from a pre-pass, and fp32 / bf16 activations are staged as a scaled fp16
// plane for the same GEMM.
int launch_gemm_w8(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec, const uint8_t* packed,
                   const float* scale, const float* bias, int64_t N, void* y, int yt, int64_t ldy, void* ws,
                   int64_t ws_bytes, hipStream_t st, bool yvec);
// split: scratch after the workspace's layout (split_area_bytes of the plan;
// a shorter or null one runs the shape without splitting K).
// Direct-to-LDS GEMM plan: block configuration id and K splits (1: none);
// with splits, `tiles` output blocks of 64 x 64 and their partial tiles.
struct DlPlan {
  int id, splits;
  int64_t tiles, part_bytes;
};
DlPlan plan_gemm_dl(bool i8, int xt, int64_t M, int64_t Nt, int64_t Kc, bool rsp);
// Bytes of a plan's split-K scratch (0 without splits): tile counters, then
// the partial tiles; the GEMM launchers take it after their other scratch.
int64_t split_area_bytes(const DlPlan& p);

// W-only prefill scratch: [rowsum: M floats][rscale: M floats][fp16 plane: M x K for
// fp32 and bf16 x, none for fp16], each part 256-byte aligned.
struct W8Ws {
  int64_t rowsum, rscale, planes, bytes;
};
W8Ws w8_ws_layout(int64_t M, int64_t K, int xt);
// Per-token symmetric W8A8 (opt-in int8-dyn granularity): xq scratch M x Kp
// bytes (Kp = ceil(K/64)*64), s_t scratch M floats.
int launch_gemm_w8a8_token(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec,
                           const uint8_t* packed, const float* scale, const float* bias, int64_t N, void* y, int yt,
                           int64_t ldy, int32_t* acc_out, int8_t* xq, float* s_t, hipStream_t st, bool yvec);
// uint8 xq [M][ldq] of fbgemm's per-tensor activation quantization from the
// min/max partials (sbq_act_quant_per_tensor).
int launch_act_quant_u8(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec, const float2* partials,
                        int nparts, uint8_t* xq, int64_t ldq, hipStream_t st);
int launch_quantize_rows_sym(const void* x, int xt, int64_t ldx, bool xvec, int64_t M, int64_t K, int64_t Kp,
                             int8_t* xq, float* s_out, hipStream_t st);
// Per-row sums in fp32 of fp16 x [M, K] (K % 8 == 0, 16-byte aligned rows).
int launch_rowsum_f16(const void* x, int64_t ldx, int64_t M, int64_t K, float* out, hipStream_t st,
                      uint32_t* zero = nullptr, int nzero = 0);
// fp32 / bf16 x [M, K] -> a scaled fp16 plane, row sums and row scales.
int launch_stage_act(const void* x, int xt, int64_t ldx, int64_t M, int64_t K, _Float16* xs, float* rowsum,
                     float* rscale, hipStream_t st, uint32_t* zero = nullptr, int nzero = 0);

// W8A8 (fbgemm dynamic semantics).  Both launch the activation min/max
// pre-pass into `partials` (>= kMinMaxPartials float2) when they need it (the
// decode fast path reduces a small x in the kernel instead).
int launch_gemv_w8a8(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec, const uint8_t* packed,
                     const float* scale, const int32_t* colsum, const float* bias, int64_t N, void* y, int yt,
                     int64_t ldy, int32_t* acc_out, float2* partials, hipStream_t st, bool yvec,
                     GemvArgmaxOut* am = nullptr);
// The GEMM quantizes x once into xq (s8 [M][Kc*64]) and writes (s_x, zp) to
// qpbuf[0..1] (zp as int bits) before the tiled pipeline reads them.
int launch_gemm_w8a8(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, bool xvec, const uint8_t* packed,
                     const float* scale, const int32_t* colsum, const float* bias, int64_t N, void* y, int yt,
                     int64_t ldy, int32_t* acc_out, float2* partials, int8_t* xq, float* qpbuf, hipStream_t st,
                     bool yvec, uint8_t* split = nullptr, int64_t split_bytes = 0);

}  // namespace sbq

// sbq_abi.hip - the extern "C" entry points of libsbq.so (declared in
// include/sbq.h).  Argument validation and kernel selection only: no device
// allocation, no mutable global state, every call asynchronous on the given
// stream.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <mutex>

#include "sbq.h"
#include "sbq_common.h"
#include "sbq_gemv_ops.h"
#include "sbq_launch.h"

namespace {

constexpr int64_t kIntMax = 0x7fffffff;

inline bool valid_dtype(int t) { return t == SBQ_F32 || t == SBQ_F16 || t == SBQ_BF16; }
inline int64_t esize(int t) { return t == SBQ_F32 ? 4 : 2; }
inline bool aligned(const void* p, int64_t a) { return ((uintptr_t)p % (uintptr_t)a) == 0; }

// Common shape / pointer checks of the linear entry points.
int check_linear(const void* x, int xt, int64_t M, int64_t K, int64_t ldx, const void* packed, const float* scale,
                 int64_t N, const void* y, int yt, int64_t ldy) {
  if (!valid_dtype(xt) || !valid_dtype(yt)) return SBQ_ERR_DTYPE;
  if (M < 0 || N < 1 || K < 1 || M > kIntMax || N > kIntMax || K > kIntMax) return SBQ_ERR_ARG;
  if (M == 0) return SBQ_OK;
  if (ldx < K || ldy < N) return SBQ_ERR_ARG;
  if (!x || !packed || !scale || !y) return SBQ_ERR_ARG;
  if (!aligned(packed, 16)) return SBQ_ERR_ALIGN;
  return SBQ_OK;
}

inline bool x_vec_ok(const void* x, int xt, int64_t ldx) {
  return aligned(x, 16) && (ldx * esize(xt)) % 16 == 0;
}
inline bool y_vec_ok(const void* y, int yt, int64_t ldy, int64_t N) {
  const int64_t a = 4 * esize(yt);
  return aligned(y, a) && (ldy * esize(yt)) % a == 0 && N % 4 == 0;
}

// W8A8 workspace layout (from the first 256-byte boundary): min/max partials
// (kMinMaxPartials float2), then (s_x, zp) in 256 bytes, then the quantized
// activations xq [M][Kc*64] (s8) for the GEMM path.
constexpr int64_t kWsPartialBytes = 256 * 8;
constexpr int64_t kWsQpBytes = 256;
inline float2* ws_partials(void* workspace) {
  return (float2*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
}
inline float* ws_qp(void* workspace) { return (float*)((uint8_t*)ws_partials(workspace) + kWsPartialBytes); }
inline int8_t* ws_xq(void* workspace) { return (int8_t*)((uint8_t*)ws_qp(workspace) + kWsQpBytes); }
// per-token scales after the quantized activations
inline float* ws_stok(void* workspace, int64_t M, int64_t K) {
  const int64_t xq = M * (((K + 63) / 64) * 64);
  return (float*)((uint8_t*)ws_xq(workspace) + ((xq + 255) & ~(int64_t)255));
}

// The int8-dyn path of one call as the entry points below run it: scratch
// from a caller's workspace or from the no-allocation array.
// Whether the int8-dyn GEMM of an [M, N, K] call can run its planned
// configuration with `split_bytes` of split-K area (its mid-sized-M plan is
// then the alternative to the row-tile GEMV).
bool w8a8_gemm_alt(int64_t M, int64_t N, int64_t K, int64_t split_bytes) {
  const sbq::DlPlan p = sbq::plan_gemm_dl(true, sbq::XT_F16, M, (N + 15) / 16, (K + 63) / 64, true);
  return p.splits == 1 || split_bytes >= sbq::split_area_bytes(p);
}

// Whether an int8-dyn call runs the row-tile GEMV after the pre-passes.
bool w8a8_runs_mt(int64_t M, int64_t N, int64_t K, int64_t split_bytes) {
  return M > 16 && sbq::gemv_mt_applies(M, ((K + 63) / 64) * 64, N, sbq::XT_S8, w8a8_gemm_alt(M, N, K, split_bytes));
}

int linear_w8a8_run(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* packed,
                    const float* scale, const int32_t* colsum, const float* bias, int64_t N, void* y, int y_dtype,
                    int64_t ldy, int32_t* acc_out, float2* parts, float* qp, int8_t* xq, uint8_t* split,
                    int64_t split_bytes, hipStream_t st) {
  const bool xv = x_vec_ok(x, x_dtype, ldx), yv = y_vec_ok(y, y_dtype, ldy, N);
  // 16 < M <= 64 where the row-tile GEMV applies: the pre-passes, then that
  // GEMV on the s8 rows (inside launch_gemm_w8a8) instead of the general GEMV
  const bool mt = w8a8_runs_mt(M, N, K, split ? split_bytes : 0);
  if (!mt && sbq::gemv_supports(M, K, true, x_dtype))
    return sbq::launch_gemv_w8a8(x, x_dtype, M, K, ldx, xv, packed, scale, colsum, bias, N, y, y_dtype, ldy, acc_out,
                                 parts, st, yv);
  return sbq::launch_gemm_w8a8(x, x_dtype, M, K, ldx, xv, packed, scale, colsum, bias, N, y, y_dtype, ldy, acc_out,
                               parts, xq, qp, st, yv, split, split_bytes);
}

// The split-K area after a W8A8 workspace's layout, and its bytes.
inline uint8_t* ws_split(void* workspace, int64_t M, int64_t K) {
  return (uint8_t*)ws_stok(workspace, M, K) + ((M * 4 + 255) & ~(int64_t)255);
}
inline int64_t ws_split_bytes(void* workspace, size_t workspace_bytes, int64_t M, int64_t K) {
  return (int64_t)workspace_bytes - (int64_t)(ws_split(workspace, M, K) - (uint8_t*)workspace);
}

// ---------------------------------------------------------------------------
// Scratch of sbq_linear_w8a8_noalloc: one static array per GPU (each device
// that loads the library holds its own copy until the process ends), laid out
// as the workspace of sbq_linear_w8a8 from its first 256-byte boundary: the
// activation min/max partials, (s_x, zp), then the quantized activations.
// Host code never passes the array's name to a kernel (on the host it is a
// stand-in, not a device address): the device address comes from
// hipGetSymbolAddress with that device current, kept per device once a
// lookup has succeeded.
// ---------------------------------------------------------------------------
constexpr int64_t kNoAllocHead = kWsPartialBytes + kWsQpBytes;
static_assert(kNoAllocHead % 256 == 0, "xq starts 256-byte aligned");
__device__ __align__(256) uint8_t scratch[kNoAllocHead + SBQ_NOALLOC_XQ_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];  // null until a lookup on that device succeeded

// Device address of this GPU's scratch array (the current device's).  Only
// a successful lookup is kept: a failed one (for instance a first call made
// while the stream is being captured, where the runtime may refuse the
// query) returns SBQ_ERR_LAUNCH and the next call looks again.
int scratch_ptr(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return SBQ_ERR_DEVICE;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      (void)hipGetLastError();  // clear the sticky error state of the failed query
      return SBQ_ERR_LAUNCH;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SBQ_OK;
}

static_assert(sbq::kArgmaxStateBytes <= SBQ_ARGMAX_WS_BYTES, "argmax state fits the documented size");

}  // namespace

extern "C" {

const char* sbq_version(void) { return "sbq 0.1.0 gfx950"; }

const char* sbq_status_string(int status) {
  switch (status) {
    case SBQ_OK: return "ok";
    case SBQ_ERR_ARG: return "invalid argument (size, stride or null pointer)";
    case SBQ_ERR_DTYPE: return "unsupported dtype";
    case SBQ_ERR_ALIGN: return "pointer not 16-byte aligned";
    case SBQ_ERR_WORKSPACE: return "workspace missing or too small";
    case SBQ_ERR_LAUNCH: return "HIP kernel launch failed";
    case SBQ_ERR_DEVICE: return "current device is not gfx950";
  }
  return "unknown status";
}

int sbq_check_device(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return SBQ_ERR_DEVICE;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return SBQ_ERR_DEVICE;
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? SBQ_OK : SBQ_ERR_DEVICE;
}

int sbq_quantize_per_channel(const void* w, int w_dtype, int64_t N, int64_t K, int64_t ldw, int8_t* q, int64_t ldq,
                             float* scale, void* stream) {
  if (!valid_dtype(w_dtype)) return SBQ_ERR_DTYPE;
  if (N < 0 || K < 1 || ldw < K || ldq < K || N > kIntMax || K > kIntMax) return SBQ_ERR_ARG;
  if (N == 0) return SBQ_OK;
  if (!w || !q || !scale) return SBQ_ERR_ARG;
  return sbq::launch_quantize_per_channel(w, w_dtype, N, K, ldw, q, ldq, scale, (hipStream_t)stream);
}

int64_t sbq_packed_bytes(int64_t N, int64_t K) {
  if (N < 1 || K < 1) return 0;
  return ((N + 15) / 16) * 16 * ((K + 63) / 64) * 64;
}

int sbq_repack_w8(const int8_t* q, int64_t N, int64_t K, int64_t ldq, uint8_t* packed, int32_t* colsum,
                  void* stream) {
  if (N < 1 || K < 1 || ldq < K || N > kIntMax || K > kIntMax) return SBQ_ERR_ARG;
  if (!q || !packed) return SBQ_ERR_ARG;
  if (!aligned(packed, 16)) return SBQ_ERR_ALIGN;
  return sbq::launch_repack(q, N, K, ldq, packed, colsum, (hipStream_t)stream);
}

int sbq_unpack_w8(const uint8_t* packed, int64_t N, int64_t K, int8_t* q, int64_t ldq, void* stream) {
  if (N < 1 || K < 1 || ldq < K || N > kIntMax || K > kIntMax) return SBQ_ERR_ARG;
  if (!q || !packed) return SBQ_ERR_ARG;
  return sbq::launch_unpack(packed, N, K, q, ldq, (hipStream_t)stream);
}

int64_t sbq_w8_workspace_bytes(int64_t M, int64_t K, int x_dtype) {
  if (M < 0 || K < 0 || M > kIntMax || K > kIntMax || !valid_dtype(x_dtype)) return 0;
  return 256 + sbq::w8_ws_layout(M, ((K + 63) / 64) * 64, x_dtype).bytes;
}

int sbq_linear_w8(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* packed,
                  const float* scale, const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy,
                  void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_linear(x, x_dtype, M, K, ldx, packed, scale, N, y, y_dtype, ldy);
  if (rc || M == 0) return rc;
  const bool xv = x_vec_ok(x, x_dtype, ldx), yv = y_vec_ok(y, y_dtype, ldy, N);
  hipStream_t st = (hipStream_t)stream;
  if (M > 16 && M <= 64) {  // several 16-row tiles of x against streamed weights
    // the tiled GEMM's mid-sized-M plan needs the full workspace (row sums, split area)
    const bool alt = workspace && (int64_t)workspace_bytes >= sbq_linear_workspace_bytes(M, N, K, x_dtype, 0);
    const int rc =
        sbq::launch_gemv_w8_mt(x, x_dtype, M, K, ldx, xv, packed, scale, bias, N, y, y_dtype, ldy, st, yv, alt);
    if (rc != -1) return rc;
  }
  if (sbq::gemv_supports(M, K, false, x_dtype)) return sbq::launch_gemv_w8(x, x_dtype, M, K, ldx, xv, packed, scale, bias, N, y, y_dtype, ldy, st, yv);
  // optional scratch of the prefill GEMM (row sums, staged activations), 256-byte aligned
  void* ws = nullptr;
  int64_t ws_bytes = 0;
  if (workspace && (int64_t)workspace_bytes >= sbq_w8_workspace_bytes(M, K, x_dtype)) {
    ws = (void*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
    ws_bytes = (int64_t)workspace_bytes - (int64_t)((uintptr_t)ws - (uintptr_t)workspace);
  }
  return sbq::launch_gemm_w8(x, x_dtype, M, K, ldx, xv, packed, scale, bias, N, y, y_dtype, ldy, ws, ws_bytes, st,
                             yv);
}

int sbq_linear_w8_grouped(int count, const void* const* x, const int64_t* ldx, int x_dtype, int64_t M, int64_t K,
                          const uint8_t* const* packed, const float* const* scale, const float* const* bias,
                          const int64_t* N, void* const* y, const int64_t* ldy, int y_dtype, void* stream) {
  if (count < 1 || count > SBQ_MAX_GROUP || !x || !ldx || !packed || !scale || !N || !y || !ldy) return SBQ_ERR_ARG;
  static_assert(SBQ_MAX_GROUP == sbq::kGemvMaxSeg, "one segment per linear");
  bool xv = true, yv = true;
  for (int i = 0; i < count; ++i) {
    const int rc = check_linear(x[i], x_dtype, M, K, ldx[i], packed[i], scale[i], N[i], y[i], y_dtype, ldy[i]);
    if (rc) return rc;
    if (M > 0) {
      xv = xv && x_vec_ok(x[i], x_dtype, ldx[i]);
      yv = yv && y_vec_ok(y[i], y_dtype, ldy[i], N[i]);
    }
  }
  if (M == 0) return SBQ_OK;
  hipStream_t st = (hipStream_t)stream;
  if (count > 1 && sbq::gemv_supports(M, K, false, x_dtype)) {
    sbq::GemvSeg segs[SBQ_MAX_GROUP] = {};
    for (int i = 0; i < count; ++i) {
      segs[i].x = x[i];
      segs[i].packed = packed[i];
      segs[i].scale = scale[i];
      segs[i].bias = bias ? bias[i] : nullptr;
      segs[i].y = y[i];
      segs[i].ldx = ldx[i];
      segs[i].ldy = ldy[i];
      segs[i].N = (int)N[i];
      segs[i].Nt = (int)((N[i] + 15) / 16);
    }
    const int rc = sbq::launch_gemv_w8_grouped(segs, count, x_dtype, M, K, xv, y_dtype, yv, st);
    if (rc != -1) return rc;
  }
  for (int i = 0; i < count; ++i) {  // one by one: the shapes the grouped launch does not take
    const int rc = sbq_linear_w8(x[i], x_dtype, M, K, ldx[i], packed[i], scale[i], bias ? bias[i] : nullptr, N[i],
                                 y[i], y_dtype, ldy[i], nullptr, 0, stream);
    if (rc) return rc;
  }
  return SBQ_OK;
}

int64_t sbq_w8a8_workspace_bytes(int64_t M, int64_t K) {
  static_assert(sbq::kMinMaxPartials * sizeof(float2) <= kWsPartialBytes, "partials fit");
  if (M < 0 || K < 0 || M > kIntMax || K > kIntMax) return 0;
  const int64_t xq = M * (((K + 63) / 64) * 64);
  return 256 + kWsPartialBytes + kWsQpBytes + ((xq + 255) & ~(int64_t)255) + ((M * 4 + 255) & ~(int64_t)255);
}

// Whether a call of this shape reaches the tiled GEMM (the entry points'
// dispatch for 16-byte aligned rows and the full workspace): otherwise a
// decode GEMV (M <= 16, the general GEMV up to 32 tokens) or the row-tile
// GEMV (16 < M <= 64 on narrow layers) runs it.
bool runs_tiled_gemm(int64_t M, int64_t N, int64_t K, int x_dtype, bool w8a8) {
  const sbq::DlPlan p = sbq::plan_gemm_dl(w8a8, sbq::XT_F16, M, (N + 15) / 16, (K + 63) / 64, true);
  if (w8a8) {
    if (w8a8_runs_mt(M, N, K, sbq::split_area_bytes(p))) return false;
    return !sbq::gemv_supports(M, K, true, x_dtype);
  }
  if (M > 16 && M <= 64 && (x_dtype == SBQ_F16 || x_dtype == SBQ_BF16) && sbq::gemv_mt_applies(M, K, N, x_dtype, true))
    return false;
  return !sbq::gemv_supports(M, K, false, x_dtype);
}

int64_t sbq_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int x_dtype, int w8a8) {
  if (M < 0 || N < 1 || K < 1 || M > kIntMax || N > kIntMax || K > kIntMax || !valid_dtype(x_dtype)) return 0;
  if (w8a8 != 0 && w8a8 != 1) return 0;
  const int64_t Nt = (N + 15) / 16, Kc = (K + 63) / 64;
  const int64_t base = w8a8 ? sbq_w8a8_workspace_bytes(M, K) : sbq_w8_workspace_bytes(M, K, x_dtype);
  if (M == 0 || !runs_tiled_gemm(M, N, K, x_dtype, w8a8 != 0)) return base;
  // the GEMM's operands are s8 (W8A8) or fp16 (weight-only, fp32 / bf16 staged as an fp16 plane)
  return base + sbq::split_area_bytes(sbq::plan_gemm_dl(w8a8 != 0, 1, M, Nt, Kc, true));
}

int sbq_gemv_config(int64_t M, int64_t K, int x_dtype, int w8a8, int32_t* info) {
  if (!valid_dtype(x_dtype)) return SBQ_ERR_DTYPE;
  if (M < 1 || K < 1 || M > kIntMax || K > kIntMax || (w8a8 != 0 && w8a8 != 1) || !info) return SBQ_ERR_ARG;
  return sbq::gemv_config_info(M, K, w8a8 != 0, x_dtype, info);
}

int sbq_gemm_config(int64_t M, int64_t N, int64_t K, int x_dtype, int w8a8, int* splits) {
  if (!valid_dtype(x_dtype)) return SBQ_ERR_DTYPE;
  if (M < 1 || N < 1 || K < 1 || M > kIntMax || N > kIntMax || K > kIntMax || (w8a8 != 0 && w8a8 != 1))
    return SBQ_ERR_ARG;
  // with that workspace every activation dtype reaches the GEMM as fp16 (W-only:
  // fp32 / bf16 staged as an fp16 plane, row sums precomputed) or s8 (W8A8)
  const sbq::DlPlan p = sbq::plan_gemm_dl(w8a8 != 0, sbq::XT_F16, M, (N + 15) / 16, (K + 63) / 64, true);
  if (splits) *splits = runs_tiled_gemm(M, N, K, x_dtype, w8a8 != 0) ? p.splits : 0;
  return p.id;
}

int sbq_act_qparams(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, float* scale_out,
                    int32_t* zp_out, void* workspace, size_t workspace_bytes, void* stream) {
  if (!valid_dtype(x_dtype)) return SBQ_ERR_DTYPE;
  if (M < 1 || K < 1 || ldx < K || M > kIntMax || K > kIntMax) return SBQ_ERR_ARG;
  if (!x || !scale_out || !zp_out) return SBQ_ERR_ARG;
  if (!workspace || (int64_t)workspace_bytes < sbq_w8a8_workspace_bytes(M, K)) return SBQ_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  float2* parts = ws_partials(workspace);
  const int np = sbq::minmax_nparts(M, K);
  int rc = sbq::launch_minmax_partials(x, x_dtype, M, K, ldx, parts, np, st);
  if (rc) return rc;
  return sbq::launch_qparams(parts, np, scale_out, zp_out, st);
}

int sbq_act_quant_per_tensor(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* xq, int64_t ldq,
                             float* scale_out, int32_t* zp_out, void* workspace, size_t workspace_bytes,
                             void* stream) {
  if (!valid_dtype(x_dtype)) return SBQ_ERR_DTYPE;
  if (M < 1 || K < 1 || ldx < K || ldq < K || M > kIntMax || K > kIntMax) return SBQ_ERR_ARG;
  if (M * ((K + 7) / 8) > (int64_t)0x7fffffff * 256) return SBQ_ERR_ARG;  // one thread per 8 values
  if (!x || !xq || !scale_out || !zp_out) return SBQ_ERR_ARG;
  if (!workspace || (int64_t)workspace_bytes < sbq_w8a8_workspace_bytes(M, K)) return SBQ_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  float2* parts = ws_partials(workspace);
  const int np = sbq::minmax_nparts(M, K);
  int rc = sbq::launch_minmax_partials(x, x_dtype, M, K, ldx, parts, np, st);
  if (rc) return rc;
  rc = sbq::launch_qparams(parts, np, scale_out, zp_out, st);
  if (rc) return rc;
  return sbq::launch_act_quant_u8(x, x_dtype, M, K, ldx, x_vec_ok(x, x_dtype, ldx), parts, np, xq, ldq, st);
}

int sbq_linear_w8a8_token(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* packed,
                          const float* scale, const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy,
                          int32_t* acc_out, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_linear(x, x_dtype, M, K, ldx, packed, scale, N, y, y_dtype, ldy);
  if (rc || M == 0) return rc;
  if (!workspace || (int64_t)workspace_bytes < sbq_w8a8_workspace_bytes(M, K)) return SBQ_ERR_WORKSPACE;
  const bool xv = x_vec_ok(x, x_dtype, ldx), yv = y_vec_ok(y, y_dtype, ldy, N);
  return sbq::launch_gemm_w8a8_token(x, x_dtype, M, K, ldx, xv, packed, scale, bias, N, y, y_dtype, ldy, acc_out,
                                     ws_xq(workspace), ws_stok(workspace, M, K), (hipStream_t)stream, yv);
}

int sbq_linear_w8a8(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* packed,
                    const float* scale, const int32_t* colsum, const float* bias, int64_t N, void* y, int y_dtype,
                    int64_t ldy, int32_t* acc_out, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_linear(x, x_dtype, M, K, ldx, packed, scale, N, y, y_dtype, ldy);
  if (rc || M == 0) return rc;
  if (!colsum) return SBQ_ERR_ARG;
  if (!workspace || (int64_t)workspace_bytes < sbq_w8a8_workspace_bytes(M, K)) return SBQ_ERR_WORKSPACE;
  return linear_w8a8_run(x, x_dtype, M, K, ldx, packed, scale, colsum, bias, N, y, y_dtype, ldy, acc_out,
                         ws_partials(workspace), ws_qp(workspace), ws_xq(workspace), ws_split(workspace, M, K),
                         ws_split_bytes(workspace, workspace_bytes, M, K), (hipStream_t)stream);
}

int sbq_linear_w8a8_grouped(int count, const void* const* x, const int64_t* ldx, int x_dtype, int64_t M, int64_t K,
                            const uint8_t* const* packed, const float* const* scale, const int32_t* const* colsum,
                            const float* const* bias, const int64_t* N, void* const* y, const int64_t* ldy,
                            int y_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  if (count < 1 || count > SBQ_MAX_GROUP || !x || !ldx || !packed || !scale || !colsum || !N || !y || !ldy)
    return SBQ_ERR_ARG;
  bool xv = true, yv = true;
  for (int i = 0; i < count; ++i) {
    const int rc = check_linear(x[i], x_dtype, M, K, ldx[i], packed[i], scale[i], N[i], y[i], y_dtype, ldy[i]);
    if (rc) return rc;
    if (M > 0) {
      if (!colsum[i]) return SBQ_ERR_ARG;
      xv = xv && x_vec_ok(x[i], x_dtype, ldx[i]);
      yv = yv && y_vec_ok(y[i], y_dtype, ldy[i], N[i]);
    }
  }
  if (M == 0) return SBQ_OK;
  if (!workspace || (int64_t)workspace_bytes < sbq_w8a8_workspace_bytes(M, K)) return SBQ_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  if (count > 1 && sbq::gemv_supports(M, K, true, x_dtype)) {
    sbq::GemvSeg segs[SBQ_MAX_GROUP] = {};
    for (int i = 0; i < count; ++i) {
      segs[i].x = x[i];
      segs[i].packed = packed[i];
      segs[i].scale = scale[i];
      segs[i].bias = bias ? bias[i] : nullptr;
      segs[i].colsum = colsum[i];
      segs[i].y = y[i];
      segs[i].ldx = ldx[i];
      segs[i].ldy = ldy[i];
      segs[i].N = (int)N[i];
      segs[i].Nt = (int)((N[i] + 15) / 16);
    }
    const int rc = sbq::launch_gemv_w8_grouped(segs, count, x_dtype, M, K, xv, y_dtype, yv, st, true);
    if (rc != -1) return rc;
  }
  // one by one (stream order lets the calls share the workspace)
  for (int i = 0; i < count; ++i) {
    const int rc = sbq_linear_w8a8(x[i], x_dtype, M, K, ldx[i], packed[i], scale[i], colsum[i], bias ? bias[i] : nullptr,
                                   N[i], y[i], y_dtype, ldy[i], nullptr, workspace, workspace_bytes, stream);
    if (rc) return rc;
  }
  return SBQ_OK;
}

int sbq_linear_w8a8_noalloc(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* packed,
                            const float* scale, const int32_t* colsum, const float* bias, int64_t N, void* y,
                            int y_dtype, int64_t ldy, int32_t* acc_out, void* stream) {
  int rc = check_linear(x, x_dtype, M, K, ldx, packed, scale, N, y, y_dtype, ldy);
  if (rc || M == 0) return rc;
  if (!colsum) return SBQ_ERR_ARG;
  if (M * (((K + 63) / 64) * 64) > SBQ_NOALLOC_XQ_BYTES) return SBQ_ERR_WORKSPACE;
  void* s = nullptr;
  rc = scratch_ptr(&s);
  if (rc) return rc;
  // every scratch byte a call reads is written earlier in the same call (the
  // partials by the min/max pass, (s_x, zp) and xq by the quantizer), so
  // nothing is cleared between calls
  uint8_t* base = (uint8_t*)s;
  return linear_w8a8_run(x, x_dtype, M, K, ldx, packed, scale, colsum, bias, N, y, y_dtype, ldy, acc_out,
                         (float2*)base, (float*)(base + kWsPartialBytes), (int8_t*)(base + kNoAllocHead), nullptr, 0,
                         (hipStream_t)stream);
}

int sbq_linear_w8_argmax(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* packed,
                         const float* scale, const float* bias, int64_t N, float* y, int64_t ldy, int64_t* idx,
                         void* workspace, size_t workspace_bytes, void* argmax_ws, void* stream) {
  int rc = check_linear(x, x_dtype, M, K, ldx, packed, scale, N, y, SBQ_F32, ldy);
  if (rc || M == 0) return rc;
  if (!idx || !argmax_ws) return SBQ_ERR_ARG;
  if (!aligned(argmax_ws, 8)) return SBQ_ERR_ALIGN;
  hipStream_t st = (hipStream_t)stream;
  sbq::GemvArgmaxOut am{(uint8_t*)argmax_ws, idx, false};
  // decode sizes: the GEMV with the token fused; larger M: the logits exactly
  // as sbq_linear_w8 computes them (its row-tile and split-K routes), then
  // the row argmax
  if (M <= 16 && sbq::gemv_supports(M, K, false, x_dtype)) {
    const bool xv = x_vec_ok(x, x_dtype, ldx), yv = y_vec_ok(y, SBQ_F32, ldy, N);
    rc = sbq::launch_gemv_w8(x, x_dtype, M, K, ldx, xv, packed, scale, bias, N, y, SBQ_F32, ldy, st, yv, &am);
  } else {
    rc = sbq_linear_w8(x, x_dtype, M, K, ldx, packed, scale, bias, N, y, SBQ_F32, ldy, workspace, workspace_bytes,
                       stream);
  }
  if (rc || am.fused) return rc;
  return sbq::launch_argmax_rows(y, M, N, ldy, idx, st);
}

int sbq_linear_w8a8_argmax(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* packed,
                           const float* scale, const int32_t* colsum, const float* bias, int64_t N, float* y,
                           int64_t ldy, int64_t* idx, void* workspace, size_t workspace_bytes, void* argmax_ws,
                           void* stream) {
  int rc = check_linear(x, x_dtype, M, K, ldx, packed, scale, N, y, SBQ_F32, ldy);
  if (rc || M == 0) return rc;
  if (!colsum || !idx || !argmax_ws) return SBQ_ERR_ARG;
  if (!aligned(argmax_ws, 8)) return SBQ_ERR_ALIGN;
  if (!workspace || (int64_t)workspace_bytes < sbq_w8a8_workspace_bytes(M, K)) return SBQ_ERR_WORKSPACE;
  const bool xv = x_vec_ok(x, x_dtype, ldx), yv = y_vec_ok(y, SBQ_F32, ldy, N);
  hipStream_t st = (hipStream_t)stream;
  sbq::GemvArgmaxOut am{(uint8_t*)argmax_ws, idx, false};
  // decode sizes: the GEMV with the token fused; larger M: sbq_linear_w8a8's
  // own routes (bit-identical logits either way), then the row argmax
  if (M <= 16 && sbq::gemv_supports(M, K, true, x_dtype))
    rc = sbq::launch_gemv_w8a8(x, x_dtype, M, K, ldx, xv, packed, scale, colsum, bias, N, y, SBQ_F32, ldy, nullptr,
                               ws_partials(workspace), st, yv, &am);
  else
    rc = sbq_linear_w8a8(x, x_dtype, M, K, ldx, packed, scale, colsum, bias, N, y, SBQ_F32, ldy, nullptr, workspace,
                         workspace_bytes, stream);
  if (rc || am.fused) return rc;
  return sbq::launch_argmax_rows(y, M, N, ldy, idx, st);
}

int sbq_argmax_rows(const float* y, int64_t M, int64_t N, int64_t ldy, int64_t* idx, void* stream) {
  if (M < 0 || N < 1 || ldy < N || N > kIntMax || M > kIntMax) return SBQ_ERR_ARG;
  if (M == 0) return SBQ_OK;
  if (!y || !idx) return SBQ_ERR_ARG;
  return sbq::launch_argmax_rows(y, M, N, ldy, idx, (hipStream_t)stream);
}

int64_t sbq_sample_workspace_bytes(int64_t M, int64_t V) {
  if (M < 0 || V < 1 || M > 65535 || V > sbq::kSampMaxVocab) return 0;
  return sbq::sample_workspace_bytes(M) + 256;  // + alignment slack
}

int sbq_sample_rows(const float* logits, int64_t M, int64_t V, int64_t ld, float temperature, int64_t top_k,
                    float top_p, const float* u, int64_t* tokens, void* workspace, size_t workspace_bytes,
                    void* stream) {
  if (M < 0 || V < 1 || ld < V || V > sbq::kSampMaxVocab || M > 65535) return SBQ_ERR_ARG;
  if (temperature != temperature || top_p != top_p) return SBQ_ERR_ARG;
  if (M == 0) return SBQ_OK;
  if (!logits || !tokens) return SBQ_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  if (temperature <= 0.0f) return sbq::launch_argmax_rows(logits, M, V, ld, tokens, st);  // engine.py:30-31
  if (!u) return SBQ_ERR_ARG;
  if (!workspace || (int64_t)workspace_bytes < sbq_sample_workspace_bytes(M, V)) return SBQ_ERR_WORKSPACE;
  void* ws = (void*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  return sbq::launch_sample_rows(logits, M, V, ld, temperature, top_k, top_p, u, tokens, ws, st);
}

}  // extern "C"

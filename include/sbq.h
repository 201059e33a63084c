/*
 * sbq.h - C ABI of the MI355X (gfx950) quantized-linear library (libsbq.so).
 *
 * This is the drop-in boundary for the quantized-linear hot path of
 * spikingbrain-cpu: the `int8` (weight-only, symmetric per-output-channel
 * int8, fp32 scales) and `int8-dyn` (W8A8 with dynamic per-tensor asymmetric
 * uint8 activations, fbgemm semantics) formats of spikingbrain_cpu/quant.py.
 *
 * Conventions (all entry points):
 *   - plain pointers and sizes only; every pointer named `d_*` or documented as
 *     "device" is HIP device memory owned by the caller.  The library never
 *     allocates device memory: scratch space is passed in as `workspace`.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     Every call is asynchronous on that stream and reentrant: the library
 *     keeps no mutable state between calls.
 *   - matrices are row-major; `ld*` is the row stride in elements.  Row and
 *     column counts (M, N, K) above 2^31 - 1 are rejected with SBQ_ERR_ARG.
 *   - return value: SBQ_OK (0) or a negative SBQ_ERR_* code; nothing throws.
 *     sbq_status_string() names a code.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   sbq_quantize_per_channel  <- spikingbrain_cpu/quant.py:25-29 quantize_per_channel
 *   sbq_repack_w8             <- spikingbrain_cpu/quant.py:33-39 Int8Linear.__init__ buffers
 *                                and quant.py:57-61 DynamicInt8Linear.__init__ (linear_prepack)
 *   sbq_linear_w8             <- spikingbrain_cpu/quant.py:41-53 Int8Linear.forward
 *   sbq_act_qparams           <- spikingbrain_cpu/quant.py:65 (the per-tensor activation
 *                                quantization parameters chosen inside
 *                                torch.ops.quantized.linear_dynamic)
 *   sbq_act_quant_per_tensor  <- spikingbrain_cpu/quant.py:65 (those parameters and the
 *                                uint8 activations linear_dynamic multiplies)
 *   sbq_linear_w8a8           <- spikingbrain_cpu/quant.py:63-66 DynamicInt8Linear.forward
 *   sbq_argmax_rows           <- spikingbrain_cpu/engine.py:30-31 (greedy sampling,
 *                                int(logits.argmax()) over the lm_head output of
 *                                model.py:447), so the logits need not leave the GPU
 *   sbq_linear_w8_argmax,     <- spikingbrain_cpu/model.py:445-447 (lm_head) and
 *   sbq_linear_w8a8_argmax       engine.py:30-31 (its greedy token) in one launch
 *   sbq_sample_rows           <- spikingbrain_cpu/engine.py:29-42 sample (temperature,
 *                                top-k, top-p and the draw) over the lm_head logits
 */
#ifndef SBQ_H_
#define SBQ_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define SBQ_OK 0
#define SBQ_ERR_ARG (-1)        /* bad size / stride / null pointer           */
#define SBQ_ERR_DTYPE (-2)      /* unsupported dtype code                      */
#define SBQ_ERR_ALIGN (-3)      /* pointer not aligned as the entry requires   */
#define SBQ_ERR_WORKSPACE (-4)  /* workspace missing or too small              */
#define SBQ_ERR_LAUNCH (-5)     /* hipLaunchKernel / HIP runtime error         */
#define SBQ_ERR_DEVICE (-6)     /* current device is not a gfx950 GPU          */

/* ---- dtype codes -------------------------------------------------------- */
#define SBQ_F32 0
#define SBQ_F16 1
#define SBQ_BF16 2

/* Library version string, e.g. "sbq 0.1.0 gfx950". */
const char* sbq_version(void);

/* Human-readable name of a status code. */
const char* sbq_status_string(int status);

/* Checks that the current HIP device is a gfx950 part the kernels were built
 * for.  Returns SBQ_OK or SBQ_ERR_DEVICE.  Optional: every compute entry point
 * reports a launch failure on its own. */
int sbq_check_device(void);

/* ---- weight quantization and packing ------------------------------------ */

/* quantize_per_channel (spikingbrain_cpu/quant.py:25-29):
 *   scale[n] = max(max_k |w[n,k]|, 1e-8f) / 127.0f      (IEEE fp32 division)
 *   q[n,k]   = clamp(rint(w[n,k] / scale[n]), -127, 127) (IEEE fp32 division,
 *                                                         round-half-even)
 * w: device [N, K] (row stride ldw) of dtype w_dtype (F32, F16 or BF16; the
 * value is widened to fp32 exactly, as weight.float() does).
 * q: device int8 [N, K] (row stride ldq).  scale: device fp32 [N]. */
int sbq_quantize_per_channel(const void* w, int w_dtype, int64_t N, int64_t K, int64_t ldw,
                             int8_t* q, int64_t ldq, float* scale, void* stream);

/* Bytes of the packed weight layout for an [N, K] int8 matrix:
 * round_up(N,16) * round_up(K,64).  The layout is a grid of 1 KiB tiles
 * [N/16][K/64]; tile (nt,kc) holds rows nt*16..+15, columns kc*64..+63, with
 * byte  lane*16 + j,  lane = g*16 + r,  equal to  q[nt*16+r][kc*64+g*16+j] ^ 0x80
 * (offset binary, padding = 0x80 i.e. q = 0).  One tile is exactly one
 * 64-lane x 16-byte wavefront load and one MFMA 16x16 operand fragment pair. */
int64_t sbq_packed_bytes(int64_t N, int64_t K);

/* Repack (the loader hook of spikingbrain_cpu/loader.py:46-51,94; the buffers of
 * quant.py:33-39 and the prepack of quant.py:57-61):
 *   q: device int8 [N, K] (row stride ldq)  ->  packed: device, sbq_packed_bytes(N,K)
 *   colsum: device int32 [N] or NULL; colsum[n] = sum_k q[n,k]  (needed by
 *   sbq_linear_w8a8 for the activation zero-point correction). */
int sbq_repack_w8(const int8_t* q, int64_t N, int64_t K, int64_t ldq,
                  uint8_t* packed, int32_t* colsum, void* stream);

/* Inverse of sbq_repack_w8: packed -> q [N, K] (row stride ldq). */
int sbq_unpack_w8(const uint8_t* packed, int64_t N, int64_t K, int8_t* q, int64_t ldq,
                  void* stream);

/* ---- int8 weight-only linear (Int8Linear.forward, quant.py:41-53) -------- */

/* y[m,n] = (sum_k x[m,k] * q[n,k]) * scale[n] (+ bias[n])
 * x: device [M, K] (row stride ldx), dtype F32, F16 or BF16.
 *    F16/BF16 inputs are used exactly (BF16 staged for the prefill GEMM: exact
 *    down to 2^28 below each row's maximum).  F32 inputs: on the decode paths
 *    (M <= 16, and the general GEMV up to 32 tokens) split into bf16 hi +
 *    remainder (relative representation error <= 2^-16); on the staged prefill
 *    path one fp16 plane of the row scaled by a power of two (11 significant
 *    bits: about 3e-4 relative L2 on the outputs).
 * packed: from sbq_repack_w8.  scale: device fp32 [N].  bias: device fp32 [N]
 * or NULL.  y: device [M, N] (row stride ldy), dtype F32, F16 or BF16.
 * Accumulation is fp32.  Routes (16-byte aligned rows, 64 | K): M <= 16 the
 * HBM-streaming MFMA GEMV; 16 < M <= 64 the row-tile GEMV on narrow layers
 * (N <= 4096 with little x to read, or wherever the workspace below is
 * missing), else the LDS-tiled MFMA GEMM; other shapes up to 32 tokens the
 * general GEMV.
 * workspace: optional (NULL, 0 is valid).  With >= sbq_w8_workspace_bytes(M,
 * K, x_dtype) bytes the prefill GEMM (K % 64 == 0, aligned rows) runs its
 * fastest path: F16 x with per-row sums from a pre-pass; BF16 / F32 x staged
 * as a power-of-two scaled fp16 plane for the same fp16 MFMA kernel; with
 * sbq_linear_workspace_bytes it also splits K over workgroups on small grids.
 * Without it, F16 / BF16 run a slower tiled GEMM and F32 the register-staged
 * bf16 hi + lo GEMM. */
int sbq_linear_w8(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                  const uint8_t* packed, const float* scale, const float* bias, int64_t N,
                  void* y, int y_dtype, int64_t ldy,
                  void* workspace, size_t workspace_bytes, void* stream);

/* `count` (1..SBQ_MAX_GROUP) independent weight-only linears that share M, K,
 * x_dtype and y_dtype, in one launch where the decode path applies: linear i
 * is y_i = linear(x_i, packed_i, scale_i, bias_i) exactly as sbq_linear_w8
 * defines it (x_i rows of stride ldx[i], y_i [M, N[i]] of stride ldy[i]).
 * The arguments are host arrays of `count` device pointers / sizes; `bias`
 * may be NULL (no biases) or hold NULL entries.  For decode shapes (M <= 16,
 * K % 64 == 0, 16-byte aligned x rows) the linears run as one GEMV launch:
 * the launch ramp and tail of a small projection are paid once per group
 * (two 4096 x 4096 projections of different inputs: 2 x 5.1 us -> 7.5 us).
 * Otherwise each runs as sbq_linear_w8 without a workspace.  Results may differ
 * from separate sbq_linear_w8 calls in the fp32 summation order (the group is
 * tiled as one layer of its summed rows).  No counterpart in the reference:
 * it is for callers holding several independent projections of one step
 * (model.py: the two lora up-projections, the SSE and SWA output projections
 * of a hybrid layer). */
#define SBQ_MAX_GROUP 4
int sbq_linear_w8_grouped(int count, const void* const* x, const int64_t* ldx, int x_dtype,
                          int64_t M, int64_t K, const uint8_t* const* packed,
                          const float* const* scale, const float* const* bias, const int64_t* N,
                          void* const* y, const int64_t* ldy, int y_dtype, void* stream);

/* Workspace bytes that let sbq_linear_w8 run its fastest prefill path for an
 * [M, K] input of x_dtype: 2 * M floats, plus M * K * 2 bytes of staged
 * activations for BF16 and F32 x, plus alignment slack.  0 for a
 * bad argument.  No counterpart in the reference (its CPU matmul needs no
 * scratch). */
int64_t sbq_w8_workspace_bytes(int64_t M, int64_t K, int x_dtype);

/* Workspace bytes that let sbq_linear_w8 (w8a8 = 0) or sbq_linear_w8a8
 * (w8a8 = 1) run their fastest path for y [M, N] = x [M, K] * W^T with x of
 * x_dtype: the sizes of sbq_w8_workspace_bytes / sbq_w8a8_workspace_bytes
 * plus, for shapes that reach the tiled GEMM with a grid that would leave CUs
 * idle, the tile counters and fp32 / int32 partial tiles of a GEMM that
 * splits K over workgroups (its
 * last split per tile adds the partials in a fixed order, so results do not
 * depend on timing).  Those entry points split K only when given this much;
 * with the smaller sizes they run the same shapes unsplit.  0 for a bad
 * argument.  No counterpart in the reference (its CPU matmul needs no
 * scratch). */
int64_t sbq_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int x_dtype, int w8a8);

/* Plan of the tiled prefill GEMM for y [M, N] = x [M, K] * W^T with x of
 * x_dtype, as sbq_linear_w8 (w8a8 = 0) and sbq_linear_w8a8 (w8a8 = 1) run it
 * when given sbq_linear_workspace_bytes of workspace: returns the block
 * configuration id (>= 0) and stores in *splits (if not NULL) the number of
 * workgroups K is split over, or 0 when calls of this shape (16-byte aligned
 * rows, that workspace) never reach the GEMM: the decode GEMVs and the
 * row-tile GEMV run them.  Host-only: needs no GPU.
 * SBQ_ERR_ARG / SBQ_ERR_DTYPE for a bad argument.  No counterpart in the
 * reference (diagnostics and tests of the configuration choice). */
int sbq_gemm_config(int64_t M, int64_t N, int64_t K, int x_dtype, int w8a8, int* splits);

/* The general decode GEMV's configuration for an [M, K] input of x_dtype
 * (the kernel that runs ragged K, misaligned rows and 17..32 tokens on the
 * layers the row-tile GEMV leaves): info[0..8] = supported (0 / 1), row
 * tiles of x, weight tiles per group, K tiles per wave, waves per
 * workgroup, activation mode (0 registers, 1 LDS, 2 chunks), staging
 * chunks per thread, LDS bytes, and whether a kernel instance exists for
 * it.  Host-only: needs no GPU.  SBQ_ERR_ARG / SBQ_ERR_DTYPE for a bad
 * argument.  No counterpart in the reference (diagnostics and tests of the
 * configuration choice). */
int sbq_gemv_config(int64_t M, int64_t K, int x_dtype, int w8a8, int32_t* info);

/* ---- int8-dyn W8A8 linear (DynamicInt8Linear.forward, quant.py:63-66) ---- */

/* Workspace bytes sbq_linear_w8a8 / sbq_act_qparams need for an [M, K] input:
 * 2.5 KiB of activation statistics plus M * ceil(K/64)*64 bytes for the
 * quantized activations of the paths with a quantize pre-pass (M > 16), M floats of per-token
 * scales (sbq_linear_w8a8_token), plus alignment slack. */
int64_t sbq_w8a8_workspace_bytes(int64_t M, int64_t K);

/* The activation quantization parameters that fbgemm's dynamic linear chooses
 * for the whole tensor x [M, K] (uint8, qmin 0, qmax 255, no range reduction):
 *   lo = min(min x, 0), hi = max(max x, 0)
 *   scale = (double)(hi - lo) / 255, replaced by 0.1 when fp32(scale) == 0 or
 *   1/fp32(scale) overflows; scales below 6.1e-5 are raised to 6.1e-5 with
 *   lo/hi rescaled; zero_point chosen from lo or hi by the smaller error term
 *   and rounded half-even (all in double), clamped to [0, 255].
 * Results: *scale_out (device fp32[1]) and *zp_out (device int32[1]). */
int sbq_act_qparams(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                    float* scale_out, int32_t* zp_out,
                    void* workspace, size_t workspace_bytes, void* stream);

/* The activation quantization itself, the step inside
 * quantized::linear_dynamic (spikingbrain_cpu/quant.py:65) that the int8-dyn
 * entry points below fuse into their kernels: the (scale, zero_point) of
 * sbq_act_qparams, then
 *   xq[m,k] = clamp(rint(fma(x[m,k], 1/scale, zero_point)), 0, 255)
 * (one rounding, half to even) into device uint8 xq [M, K] with row stride
 * ldq >= K; sbq_linear_w8a8's acc equals sum_k (xq[m,k] - zp) * q[n,k].
 * Results: *scale_out (device fp32[1]), *zp_out (device int32[1]).
 * workspace: >= sbq_w8a8_workspace_bytes(M, K) bytes. */
int sbq_act_quant_per_tensor(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                             uint8_t* xq, int64_t ldq, float* scale_out, int32_t* zp_out,
                             void* workspace, size_t workspace_bytes, void* stream);

/* y[m,n] = fp32(acc[m,n]) * fp32(s_x * scale[n]) (+ bias[n]) where
 *   xq[m,k]  = clamp(rint(fma(x[m,k], 1/s_x, zp)), 0, 255)   (one rounding)
 *   acc[m,n] = sum_k (xq[m,k] - zp) * q[n,k]                  (exact int32)
 * which is bit-exact with torch.ops.quantized.linear_dynamic (fbgemm) on the
 * same fp32 inputs.  colsum: from sbq_repack_w8 (required).
 * acc_out: device int32 [M, N] (row stride N) or NULL; when given, the raw
 * int32 accumulators are written too (the bit-exactness check).
 * workspace: >= sbq_w8a8_workspace_bytes(M, K) bytes of device memory. */
int sbq_linear_w8a8(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                    const uint8_t* packed, const float* scale, const int32_t* colsum,
                    const float* bias, int64_t N,
                    void* y, int y_dtype, int64_t ldy, int32_t* acc_out,
                    void* workspace, size_t workspace_bytes, void* stream);

/* `count` (1..SBQ_MAX_GROUP) independent int8-dyn linears of one M, K and
 * dtypes: y_i = sbq_linear_w8a8(x_i, packed_i, scale_i, colsum_i, bias_i,
 * N_i) for each i, every x_i quantized with its own (s_x, zp).  Arguments as
 * in sbq_linear_w8_grouped, plus host arrays of the column sums (required)
 * and one workspace of >= sbq_w8a8_workspace_bytes(M, K) bytes.  For decode
 * shapes whose x fits the fused GEMV (each workgroup reduces its linear's
 * min/max itself) the linears run as one launch; otherwise one by one as
 * sbq_linear_w8a8, sharing the workspace in stream order.  Bit-exact with
 * separate calls (integer accumulation).  No counterpart in the reference:
 * it is for callers holding several independent int8-dyn projections of one
 * step (model.py: the two lora up-projections, the SSE and SWA output
 * projections of a hybrid layer). */
int sbq_linear_w8a8_grouped(int count, const void* const* x, const int64_t* ldx, int x_dtype,
                            int64_t M, int64_t K, const uint8_t* const* packed,
                            const float* const* scale, const int32_t* const* colsum,
                            const float* const* bias, const int64_t* N, void* const* y,
                            const int64_t* ldy, int y_dtype, void* workspace,
                            size_t workspace_bytes, void* stream);

/* Largest quantized-activation scratch of sbq_linear_w8a8_noalloc:
 * M * ceil(K/64)*64 bytes must not exceed it (e.g. M = 2048 at K = 4096,
 * M = 512 at K = 12288). */
#define SBQ_NOALLOC_XQ_BYTES (8 << 20)

/* sbq_linear_w8a8 without a workspace: no counterpart in the reference.  It is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc); it calls no
 * allocating routine.  Same arguments, results and bit-exactness as
 * sbq_linear_w8a8.  Its scratch (activation min/max partials, (s_x, zp), the
 * quantized activations) is a static device array of 2304 bytes +
 * SBQ_NOALLOC_XQ_BYTES that each GPU the library runs on holds until the
 * process ends; the first call on a device looks up that device's copy (make
 * it outside graph capture).  Inputs with M * ceil(K/64)*64 >
 * SBQ_NOALLOC_XQ_BYTES return SBQ_ERR_WORKSPACE before any launch.  Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams, other threads) race on it.  Nothing in it needs clearing between
 * calls (each call writes every byte it reads). */
int sbq_linear_w8a8_noalloc(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                            const uint8_t* packed, const float* scale, const int32_t* colsum,
                            const float* bias, int64_t N,
                            void* y, int y_dtype, int64_t ldy, int32_t* acc_out, void* stream);

/* Per-token symmetric W8A8: an opt-in granularity with no counterpart in the
 * reference, whose int8-dyn (quant.py:63-66, sbq_linear_w8a8 above) is
 * per-tensor asymmetric; it does not reproduce the reference's outputs.  Each
 * activation row is quantized exactly as quantize_per_channel (quant.py:25-29)
 * quantizes a weight row:
 *   s_t[m] = max(max_k |x[m,k]|, 1e-8) / 127      (IEEE fp32 division)
 *   xq[m,k] = clamp(rne(x[m,k] / s_t[m]), -127, 127)
 *   acc[m,n] = sum_k xq[m,k] * q[n,k]            (int32, exact; acc_out nullable)
 *   y[m,n] = fp32(acc) * fp32(s_t[m] * scale[n]) (with a bias: one fma)
 * workspace: >= sbq_w8a8_workspace_bytes(M, K) bytes.  The row quantizer runs
 * first; then M <= 16 runs the HBM-streaming int8 MFMA GEMV on the s8 rows,
 * larger M the tiled int8 MFMA GEMM. */
int sbq_linear_w8a8_token(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                          const uint8_t* packed, const float* scale, const float* bias, int64_t N,
                          void* y, int y_dtype, int64_t ldy, int32_t* acc_out,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ---- lm_head and the greedy token in one pass ---------------------------- */

/* Bytes of the argmax state of the two entry points below. */
#define SBQ_ARGMAX_WS_BYTES 16640

/* Int8Linear.forward over the lm_head weights (model.py:445-447 ->
 * quant.py:41-53) followed by greedy token selection (engine.py:30-31,
 * int(logits.argmax())):
 *   y      = the fp32 logits [M, N] (row stride ldy), as sbq_linear_w8
 *            computes them;
 *   idx[m] = the first n with y[m, n] maximal over row m, NaN above every
 *            number (torch.argmax; the same token sbq_argmax_rows picks on y).
 * At decode sizes (M <= 16, K % 64 == 0, 16-byte aligned x rows) the token is
 * picked inside the GEMV launch (its last workgroup decodes it); other shapes
 * run sbq_linear_w8 (with the optional workspace, as there) and then
 * sbq_argmax_rows.  argmax_ws: SBQ_ARGMAX_WS_BYTES of device memory, 8-byte
 * aligned, all zero before the first call; every call leaves it zero again.
 * Calls that can overlap (other streams) need their own argmax_ws.  idx:
 * device int64 [M]. */
int sbq_linear_w8_argmax(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                         const uint8_t* packed, const float* scale, const float* bias, int64_t N,
                         float* y, int64_t ldy, int64_t* idx,
                         void* workspace, size_t workspace_bytes, void* argmax_ws, void* stream);

/* The same for DynamicInt8Linear.forward (quant.py:63-66): y as
 * sbq_linear_w8a8 computes it (bit-exact with fbgemm), then the greedy token.
 * workspace: as for sbq_linear_w8a8.  argmax_ws: as above. */
int sbq_linear_w8a8_argmax(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                           const uint8_t* packed, const float* scale, const int32_t* colsum,
                           const float* bias, int64_t N, float* y, int64_t ldy, int64_t* idx,
                           void* workspace, size_t workspace_bytes, void* argmax_ws, void* stream);

/* ---- greedy token selection (engine.py:30-31) ---- */

/* idx[m] = the first n with y[m, n] maximal over row m of fp32 y [M, N] (row
 * stride ldy); NaN ranks above every number (torch.argmax semantics).
 * idx: device int64 [M]. */
int sbq_argmax_rows(const float* y, int64_t M, int64_t N, int64_t ldy, int64_t* idx, void* stream);

/* ---- non-greedy sampling (engine.py:29-42, sample) ---- */

/* Workspace bytes of sbq_sample_rows for M rows (about 130 KB per row, for
 * any vocabulary size up to 2^23).  0 for a bad argument. */
int64_t sbq_sample_workspace_bytes(int64_t M, int64_t V);

/* tokens[m] = the engine's sample() of row m of fp32 logits [M, V] (row
 * stride ld), as spikingbrain_cpu/engine.py:29-42 computes it:
 *   temperature <= 0: the greedy token (sbq_argmax_rows; u and the workspace
 *     may be NULL);
 *   z = logits / temperature (fp32 division); top_k > 0: tokens below the
 *     min(top_k, V)-th largest z are masked; p = softmax(z);
 *   0 < top_p < 1: a token is kept while the probability mass of the tokens
 *     above it stays below top_p, the tokens taken in the order of z (of
 *     two tokens of equal fp32 probability the larger z first; the
 *     reference's sort leaves their order open); of tokens of equal z at
 *     that boundary, as many as the rule admits, first in vocabulary order
 *     (a stable sort's order);
 *   the draw: the first index (vocabulary order) whose prefix of kept mass
 *     exceeds u[m] * (kept mass), u: device fp32 [M] uniforms in [0, 1), one
 *     per row, drawn by the caller (torch.multinomial's distribution; the
 *     caller's generator supplies the randomness).
 * Masses are exact sums of the fp32 probabilities truncated to 2^-40, so the
 * result does not depend on timing.  A row with a NaN, or an infinite
 * maximum after the division (where the reference raises), gets token -1.
 * tokens: device int64 [M].  M <= 65535, V <= 2^23 (a row's mass, at most
 * V * 2^40, fits 64 bits).  Rows are independent. */
int sbq_sample_rows(const float* logits, int64_t M, int64_t V, int64_t ld, float temperature, int64_t top_k,
                    float top_p, const float* u, int64_t* tokens, void* workspace, size_t workspace_bytes,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SBQ_H_ */

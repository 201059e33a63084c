/*
 * sbq_oracle.c - CPU restatement of spikingbrain-cpu's quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the oracle that the HIP kernels are
 * compared against; it is never linked into libsbq.so and never runs on the
 * product path.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.
 *
 * Each function cites the reference file:line it restates (paths relative to
 * the reference repository).  The `int8-dyn` format delegates its arithmetic to
 * a third-party library that is not vendored in the reference: fbgemm, as
 * bundled in the torch wheel the reference pins (requirements.txt:2,
 * torch==2.14.1+cpu), reached through torch.ops.quantized.linear_dynamic
 * (quant.py:65) with PyTorch's ChooseQuantizationParams
 * (aten/src/ATen/native/quantized/cpu/QuantUtils.h) choosing the activation
 * parameters.  The restatement below is that published algorithm; it is
 * pinned bit-exactly against the live torch op by tests/test_oracle.py.
 *
 * Build: oracle/Makefile -> oracle/_build/libsbq_oracle.so (gcc -O2, no
 * -ffast-math, no FMA contraction: every rounding below is explicit).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

/* quant.py:25-29  quantize_per_channel
 *   w = weight.float(); scale = w.abs().amax(dim=1).clamp(min=1e-8) / 127.0
 *   q = torch.round(w / scale[:, None]).clamp(-127, 127).to(torch.int8)
 * fp32 IEEE division for both divisions, round-half-even (rintf under the
 * default rounding mode). */
void oracle_quantize_per_channel(const float* w, int64_t N, int64_t K, int8_t* q, float* scale) {
  for (int64_t n = 0; n < N; ++n) {
    const float* row = w + n * K;
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      float a = fabsf(row[k]);
      if (a > amax) amax = a;
    }
    float clamped = amax < 1e-8f ? 1e-8f : amax;
    volatile float s = clamped / 127.0f;
    scale[n] = s;
    for (int64_t k = 0; k < K; ++k) {
      volatile float t = row[k] / s;
      float r = rintf(t);
      if (r > 127.0f) r = 127.0f;
      if (r < -127.0f) r = -127.0f;
      q[n * K + k] = (int8_t)r;
    }
  }
}

/* quant.py:41-53  Int8Linear.forward
 *   x2 = x.reshape(-1, K).float()
 *   out = cat_blocks(x2 @ qweight[blk].float().t()) * scale (+ bias)
 * The dot product is accumulated in double (exact for these magnitudes up to
 * the final rounding), rounded once to fp32, then multiplied by the per-row
 * scale in fp32 - the scale is applied after the dot product, as quant.py:50
 * does.  The reference's sgemm accumulates in fp32 in an unspecified order;
 * comparisons against either use a relative-L2 tolerance. */
void oracle_int8_linear(const float* x, int64_t M, int64_t K, const int8_t* q, const float* scale,
                        const float* bias, int64_t N, float* y) {
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0;
      const float* xr = x + m * K;
      const int8_t* qr = q + n * K;
      for (int64_t k = 0; k < K; ++k) acc += (double)xr[k] * (double)qr[k];
      volatile float a32 = (float)acc;
      volatile float out = a32 * scale[n];
      if (bias) out = out + bias[n];
      y[m * N + n] = out;
    }
  }
}

/* fbgemm dynamic activation parameters (quant.py:65 -> linear_dynamic ->
 * ChooseQuantizationParams(min, max, qmin=0, qmax=255, preserve_sparsity=false,
 * force_scale_power_of_two=false, reduce_range=false)). */
void oracle_choose_qparams(float xmin, float xmax, float* scale_out, int32_t* zp_out) {
  const int32_t qmin = 0, qmax = 255;
  const float SMALL_SCALE_THRESHOLD = 6.1e-5f;
  float lo = xmin < 0.0f ? xmin : 0.0f;
  float hi = xmax > 0.0f ? xmax : 0.0f;
  double scale = ((double)hi - (double)lo) / (double)(qmax - qmin);
  volatile float fs = (float)scale;
  volatile float inv = 1.0f / fs;
  if (fs == 0.0f || isinf(inv)) scale = 0.1;
  if (scale < (double)SMALL_SCALE_THRESHOLD) {
    float org = (float)scale;
    scale = (double)SMALL_SCALE_THRESHOLD;
    if (lo == 0.0f) {
      hi = SMALL_SCALE_THRESHOLD * (float)(qmax - qmin);
    } else if (hi == 0.0f) {
      lo = -SMALL_SCALE_THRESHOLD * (float)(qmax - qmin);
    } else {
      volatile float amp = SMALL_SCALE_THRESHOLD / org;
      lo = lo * amp;
      hi = hi * amp;
    }
  }
  double zp_from_min = (double)qmin - (double)lo / scale;
  double zp_from_max = (double)qmax - (double)hi / scale;
  double err_min = fabs((double)qmin) - fabs((double)lo / scale);
  double err_max = fabs((double)qmax) - fabs((double)hi / scale);
  double z0 = err_min < err_max ? zp_from_min : zp_from_max;
  int32_t zp;
  if (z0 < qmin) zp = qmin;
  else if (z0 > qmax) zp = qmax;
  else zp = (int32_t)nearbyint(z0);
  *scale_out = (float)scale;
  *zp_out = zp;
}

/* fbgemm Quantize<uint8_t> as used while packing A: inv = 1.0f/scale (fp32),
 * t = fma(x, inv, zp) rounded once to fp32, then round-half-even, clamp. */
void oracle_quantize_act(const float* x, int64_t n, float scale, int32_t zp, uint8_t* xq) {
  volatile float inv = 1.0f / scale;
  for (int64_t i = 0; i < n; ++i) {
    float t = fmaf(x[i], inv, (float)zp);
    float r = rintf(t);
    if (r < 0.0f) r = 0.0f;
    if (r > 255.0f) r = 255.0f;
    xq[i] = (uint8_t)r;
  }
}

/* fbgemm ReQuantizeForFloat epilogue as linear_dynamic runs it:
 *   y = fp32(acc) * fp32(s_x * scale[n])                  without bias
 *   y = fma(fp32(acc), fp32(s_x * scale[n]), bias[n])     with bias (one rounding) */
void oracle_dyn_epilogue(const int32_t* acc, int64_t M, int64_t N, float sx, const float* scale,
                         const float* bias, float* y) {
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      volatile float mult = sx * scale[n];
      float a = (float)acc[m * N + n];
      volatile float out = bias ? fmaf(a, mult, bias[n]) : a * mult;
      y[m * N + n] = out;
    }
  }
}

/* Per-token symmetric W8A8 epilogue (opt-in granularity, no counterpart in the
 * reference): y = fp32(acc) * fp32(s_t[m] * scale[n]), with a bias one fma. */
void oracle_dyn_epilogue_token(const int32_t* acc, int64_t M, int64_t N, const float* st, const float* scale,
                               const float* bias, float* y) {
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      volatile float mult = st[m] * scale[n];
      float a = (float)acc[m * N + n];
      volatile float out = bias ? fmaf(a, mult, bias[n]) : a * mult;
      y[m * N + n] = out;
    }
  }
}

/* quant.py:63-66  DynamicInt8Linear.forward == linear_dynamic(x, packed):
 *   acc[m,n] = sum_k (xq[m,k] - zp) * q[n,k]            (exact integer)
 *   y[m,n]   = oracle_dyn_epilogue(acc)
 * acc_out (int32 [M,N]) and xq_out (uint8 [M,K]) may be NULL. */
void oracle_dyn_linear(const float* x, int64_t M, int64_t K, const int8_t* q, const float* scale,
                       const float* bias, int64_t N, float* y, int32_t* acc_out, uint8_t* xq_out,
                       float* sx_out, int32_t* zp_out) {
  float xmin = x[0], xmax = x[0];
  for (int64_t i = 1; i < M * K; ++i) {
    if (x[i] < xmin) xmin = x[i];
    if (x[i] > xmax) xmax = x[i];
  }
  float sx;
  int32_t zp;
  oracle_choose_qparams(xmin, xmax, &sx, &zp);
  uint8_t* xq = xq_out ? xq_out : (uint8_t*)malloc((size_t)(M * K));
  oracle_quantize_act(x, M * K, sx, zp, xq);
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      int64_t acc = 0;
      for (int64_t k = 0; k < K; ++k) acc += ((int64_t)xq[m * K + k] - zp) * (int64_t)q[n * K + k];
      int32_t a32 = (int32_t)acc;
      if (acc_out) acc_out[m * N + n] = a32;
      oracle_dyn_epilogue(&a32, 1, 1, sx, scale + n, bias ? bias + n : NULL, y + m * N + n);
    }
  }
  if (!xq_out) free(xq);
  if (sx_out) *sx_out = sx;
  if (zp_out) *zp_out = zp;
}

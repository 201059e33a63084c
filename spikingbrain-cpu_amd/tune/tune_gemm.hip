// Tuning harness for the prefill GEMM's configuration model (pick_gemm_dl):
// runs one direct-to-LDS configuration, chosen by id, on operands the caller
// prepared with the library (packed weights, and for int8-dyn the s8 rows and
// (s_x, zp) of the quantize pre-pass; for fp16 weight-only the row sums).  It
// compiles the library's GEMM source into its own shared object, so the
// product ABI stays as include/sbq.h declares it; sweep.py drives it and
// fit.py refits the model's coefficients from what it measured.
#include "../csrc/sbq_gemm.hip"

extern "C" {

// fp16 weight-only GEMM, configuration `id`, fp16 x [M, K] (row stride ldx),
// row sums rsum [M] (launch_rowsum_f16), fp16 y [M, N].  Returns 0, or -1 when
// that configuration cannot run the shape.
int sbq_tune_gemm_w8(int id, const void* x, int64_t ldx, int M, int K, const uint8_t* packed, const float* scale,
                     int N, void* y, const float* rsum, void* stream) {
  using namespace sbq;
  if (K % 64 != 0) return -1;
  GemmArgs a{};
  a.x = x; a.ldx = ldx; a.M = M; a.Kc = K / 64; a.packed = packed; a.scale = scale;
  a.N = N; a.Nt = (N + 15) / 16; a.y = y; a.yt = XT_F16; a.ldy = N; a.rsum = rsum;
  a.flags = 1 | 2 | y16_flag(y, XT_F16, N);
  return launch_gemm_dl_cfg(id, false, XT_F16, a, (hipStream_t)stream);
}

// int8-dyn GEMM, configuration `id`, on the s8 rows xq [M, Kp] (Kp = ceil(K/64)
// * 64) and the (s_x, zp) words qp of the quantize pre-pass; fp16 y [M, N].
int sbq_tune_gemm_w8a8(int id, const void* xq, int M, int K, const uint8_t* packed, const float* scale,
                       const int32_t* colsum, int N, void* y, const float* qp, void* stream) {
  using namespace sbq;
  const int Kc = (K + 63) / 64;
  GemmArgs a{};
  a.x = xq; a.ldx = (int64_t)Kc * 64; a.M = M; a.Kc = Kc; a.packed = packed; a.scale = scale; a.colsum = colsum;
  a.N = N; a.Nt = (N + 15) / 16; a.y = y; a.yt = XT_F16; a.ldy = N; a.qpbuf = qp;
  a.flags = 2 | y16_flag(y, XT_F16, N);
  return launch_gemm_dl_cfg(id, true, XT_F16, a, (hipStream_t)stream);
}

// Either GEMM on activation rows of stride ldx (elements for fp16, bytes for
// s8), with K split over `splits` workgroups (splits > 1: configurations with
// a split instance, 3 / 15 and the mid-sized-M ones): `part` holds tiles * splits partial tiles
// of that configuration's block (BN x BM x 4 bytes) and `tcount` one counter
// per output block, zero before the first launch (each launch leaves them
// zero).  w8a8 = 0: fp16 x with row sums `aux` [M]; 1: s8 rows with the
// (s_x, zp) words `aux`.  fp16 y [M, N].
int sbq_tune_gemm_split(int w8a8, int id, int splits, const void* x, int64_t ldx, int M, int K,
                        const uint8_t* packed, const float* scale, const int32_t* colsum, int N, void* y,
                        const float* aux, uint8_t* part, uint32_t* tcount, void* stream) {
  using namespace sbq;
  if (K % 64 != 0 || splits < 1) return -1;
  GemmArgs a{};
  a.x = x; a.ldx = ldx; a.M = M; a.Kc = K / 64; a.packed = packed; a.scale = scale;
  a.N = N; a.Nt = (N + 15) / 16; a.y = y; a.yt = XT_F16; a.ldy = N;
  if (w8a8) {
    a.colsum = colsum;
    a.qpbuf = aux;
    a.flags = 2 | y16_flag(y, XT_F16, N);
  } else {
    a.rsum = aux;
    a.flags = 1 | 2 | y16_flag(y, XT_F16, N);
  }
  if (splits > 1) {
    a.part = part; a.tcount = tcount; a.splits = splits;
  }
  return launch_gemm_dl_cfg(id, w8a8 != 0, XT_F16, a, (hipStream_t)stream);
}

// The decode row-tile GEMV (16 < M <= 64, launch_gemv_mt) on fp16 x (w8a8 = 0)
// or on the s8 rows and (s_x, zp) words of the quantize pre-pass (w8a8 = 1),
// for comparing it with the tiled GEMM at the same shapes.  fp16 y [M, N].
int sbq_tune_gemv_mt(int w8a8, const void* x, int M, int K, const uint8_t* packed, const float* scale,
                     const int32_t* colsum, int N, void* y, const float* qp, void* stream) {
  using namespace sbq;
  if (K % 64 != 0) return -1;
  GemvArgs g{};
  g.x = x; g.ldx = K; g.M = M; g.K = K; g.Kc = K / 64;
  g.packed = packed; g.scale = scale; g.N = N; g.Nt = (N + 15) / 16; g.y = y; g.yt = XT_F16; g.ldy = N;
  g.flags = kGemvXVec | (N % 4 == 0 ? kGemvYVec : 0);
  if (w8a8) {
    g.colsum = colsum;
    g.qpbuf = qp;
  }
  return launch_gemv_mt(g, w8a8 ? XT_S8 : XT_F16, (hipStream_t)stream, false);
}

// Row sums of fp16 x for sbq_tune_gemm_w8.
int sbq_tune_rowsum_f16(const void* x, int64_t ldx, int M, int K, float* out, void* stream) {
  return sbq::launch_rowsum_f16(x, ldx, M, K, out, (hipStream_t)stream);
}

// The configuration the library picks (pick_gemm_dl) for M > 128.
int sbq_tune_pick(int w8a8, int M, int N, int K) {
  return sbq::pick_gemm_dl(w8a8 != 0, sbq::XT_F16, M, (N + 15) / 16, (K + 63) / 64);
}

}  // extern "C"

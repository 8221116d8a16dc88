/*
 * The C ABI driven from C, with no torch and no Python in the process: the
 * per-token quantizers and the W8A8 GEMMs of include/xgen_amd.h on hipMalloc'd
 * buffers, in the order a DiT linear calls them, checked on the host against
 * the oracle's C quantizers (oracle/quant_ref.c: bytes and scales bit-exact)
 * and against sums of the decoded operands (INT8 accumulators exact, FP8
 * accumulators within each kind's bound), plus the error contract.
 *
 * Test infrastructure: tests/c_abi/build.py builds it into tests/c_abi/_build/;
 * tests/test_gpu_c_abi.py runs it.  Exit status 0: every check passed; 77: no
 * HIP device; anything else: a failure, described on stdout.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "xgen_amd.h"

/* the oracle's C restatement (oracle/quant_ref.c) */
void oracle_quant_rows_fp8(int fmt, const uint16_t *x, int64_t rows, int64_t cols, uint8_t *q, float *scale);
void oracle_quant_rows_int8(int fmt, const uint16_t *x, int64_t rows, int64_t cols, int8_t *q, float *scale);
float oracle_e4m3_decode(uint8_t b);
float oracle_half_to_f32(int fmt, uint16_t h);

enum { M = 200, K = 384, N = 256 };  /* M off the 256-row tile, K and N multiples of 16 */

static int failures = 0;

#define EXPECT(cond, ...)            \
  do {                               \
    if (!(cond)) {                   \
      printf("FAIL: " __VA_ARGS__);  \
      printf("\n");                  \
      ++failures;                    \
    }                                \
  } while (0)

#define HIP_OK(call)                                                          \
  do {                                                                        \
    hipError_t e_ = (call);                                                   \
    if (e_ != hipSuccess) {                                                   \
      printf("FAIL: %s -> %s\n", #call, hipGetErrorString(e_));               \
      exit(1);                                                                \
    }                                                                         \
  } while (0)

#define XGEN_OK_CALL(call)                                                    \
  do {                                                                        \
    int s_ = (call);                                                          \
    if (s_ != XGEN_OK) {                                                      \
      printf("FAIL: %s -> %s: %s\n", #call, xgen_status_string(s_), xgen_last_error()); \
      exit(1);                                                                \
    }                                                                         \
  } while (0)

static uint32_t lcg = 12345u;
static float uniform(void) { /* [0, 1) */
  lcg = lcg * 1664525u + 1013904223u;
  return (float)(lcg >> 8) * (1.0f / 16777216.0f);
}
static float bell(void) { /* mean 0, variance 1: a sum of four uniforms */
  return (uniform() + uniform() + uniform() + uniform() - 2.0f) * 1.7320508f;
}

static uint16_t bf16_bits(float f) { /* round to nearest even */
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
static float bf16_value(uint16_t h) { return oracle_half_to_f32(XGEN_DTYPE_BF16, h); }

static void *device_copy(const void *host, size_t bytes) {
  void *d = NULL;
  HIP_OK(hipMalloc(&d, bytes));
  if (host) HIP_OK(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice));
  return d;
}
static void host_copy(void *host, const void *dev, size_t bytes) {
  HIP_OK(hipMemcpy(host, dev, bytes, hipMemcpyDeviceToHost));
}

int main(void) {
  int devices = 0;
  if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) {
    printf("no HIP device\n");
    return 77;
  }
  EXPECT(xgen_abi_version() == XGEN_ABI_VERSION, "abi version %d", xgen_abi_version());
  EXPECT(strcmp(xgen_status_string(XGEN_OK), "ok") == 0, "status string of XGEN_OK");

  /* activations with two x50 outlier channels, weights ~0.02, bias ~0.01 (bf16) */
  static uint16_t x[M * K], w[N * K], bias[N];
  for (int m = 0; m < M; ++m)
    for (int k = 0; k < K; ++k) x[m * K + k] = bf16_bits(bell() * ((k == 17 || k == 300) ? 50.0f : 1.0f));
  for (int i = 0; i < N * K; ++i) w[i] = bf16_bits(bell() * 0.02f);
  for (int n = 0; n < N; ++n) bias[n] = bf16_bits(bell() * 0.01f);

  hipStream_t stream;
  HIP_OK(hipStreamCreate(&stream));
  void *dx = device_copy(x, sizeof x), *dw = device_copy(w, sizeof w), *db = device_copy(bias, sizeof bias);

  /* ---- FP8: per-token / per-channel quantizers, then both GEMM kinds */
  static uint8_t qx[M * K], qw[N * K], rqx[M * K], rqw[N * K];
  static float sx[M], sw[N], rsx[M], rsw[N];
  void *dqx = device_copy(NULL, sizeof qx), *dqw = device_copy(NULL, sizeof qw);
  float *dsx = device_copy(NULL, sizeof sx), *dsw = device_copy(NULL, sizeof sw);
  XGEN_OK_CALL(xgen_quantize_rows(XGEN_DTYPE_BF16, dx, M, K, K, XGEN_DTYPE_E4M3, dqx, K, dsx, stream));
  XGEN_OK_CALL(xgen_quantize_rows(XGEN_DTYPE_BF16, dw, N, K, K, XGEN_DTYPE_E4M3, dqw, K, dsw, stream));
  HIP_OK(hipStreamSynchronize(stream));
  host_copy(qx, dqx, sizeof qx), host_copy(qw, dqw, sizeof qw);
  host_copy(sx, dsx, sizeof sx), host_copy(sw, dsw, sizeof sw);
  oracle_quant_rows_fp8(XGEN_DTYPE_BF16, x, M, K, rqx, rsx);
  oracle_quant_rows_fp8(XGEN_DTYPE_BF16, w, N, K, rqw, rsw);
  EXPECT(memcmp(qx, rqx, sizeof qx) == 0 && memcmp(sx, rsx, sizeof sx) == 0, "fp8 activation bytes / scales");
  EXPECT(memcmp(qw, rqw, sizeof qw) == 0 && memcmp(sw, rsw, sizeof sw) == 0, "fp8 weight bytes / scales");

  static float acc[M * N];
  static uint16_t out[M * N];
  float *dacc = device_copy(NULL, sizeof acc);
  void *dout = device_copy(NULL, sizeof out);
  for (int exact = 0; exact < 2; ++exact) {
    if (exact)
      XGEN_OK_CALL(xgen_scaled_mm_fp8_exact(dqx, K, dqw, K, M, N, K, dsx, 1, dsw, 1, db, XGEN_DTYPE_BF16,
                                            XGEN_ACT_NONE, dout, XGEN_DTYPE_BF16, N, dacc, stream));
    else
      XGEN_OK_CALL(xgen_scaled_mm_fp8(dqx, K, dqw, K, M, N, K, dsx, 1, dsw, 1, db, XGEN_DTYPE_BF16, XGEN_ACT_NONE,
                                      dout, XGEN_DTYPE_BF16, N, dacc, stream));
    HIP_OK(hipStreamSynchronize(stream));
    host_copy(acc, dacc, sizeof acc), host_copy(out, dout, sizeof out);
    /* exact kind: fp32 sums of exact products, within K 2^-24 sum|a w|; FP8 MFMA kind: within
       2^-11 sum|a w| (its truncation inside each group of 8 products) */
    const double bound = exact ? (double)K * ldexp(1.0, -24) : ldexp(1.0, -11);
    double worst = 0.0;
    int bad_out = 0;
    for (int m = 0; m < M; ++m)
      for (int n = 0; n < N; ++n) {
        double sum = 0.0, mag = 0.0;
        for (int k = 0; k < K; ++k) {
          const double p = (double)oracle_e4m3_decode(qx[m * K + k]) * oracle_e4m3_decode(qw[n * K + k]);
          sum += p, mag += fabs(p);
        }
        const double err = fabs(acc[m * N + n] - sum) / (mag > 0 ? mag : 1.0);
        if (err > worst) worst = err;
        /* the epilogue: bf16(acc * (sa * sw) + bias), one rounding step of slack */
        const float y = fmaf(acc[m * N + n], sx[m] * sw[n], bf16_value(bias[n]));
        const float got = bf16_value(out[m * N + n]);
        if (fabsf(got - y) > ldexpf(fabsf(y), -8) + 1e-30f) ++bad_out;
      }
    EXPECT(worst <= bound, "fp8 %s accumulators: worst |acc - sum| / sum|a w| = %.3g > %.3g",
           exact ? "exact" : "mfma", worst, bound);
    EXPECT(bad_out == 0, "fp8 %s outputs: %d off the epilogue of the accumulators", exact ? "exact" : "mfma",
           bad_out);
  }

  /* ---- INT8: quantizers, then the GEMM with its int32 accumulators */
  static int8_t ix[M * K], iw[N * K], rix[M * K], riw[N * K];
  static int32_t iacc[M * N];
  void *dix = device_copy(NULL, sizeof ix), *diw = device_copy(NULL, sizeof iw);
  int32_t *diacc = device_copy(NULL, sizeof iacc);
  XGEN_OK_CALL(xgen_quantize_rows(XGEN_DTYPE_BF16, dx, M, K, K, XGEN_DTYPE_I8, dix, K, dsx, stream));
  XGEN_OK_CALL(xgen_quantize_rows(XGEN_DTYPE_BF16, dw, N, K, K, XGEN_DTYPE_I8, diw, K, dsw, stream));
  XGEN_OK_CALL(xgen_quant_matmul_int8(dix, K, diw, K, M, N, K, dsx, 1, dsw, 1, db, XGEN_DTYPE_BF16, XGEN_ACT_NONE,
                                      dout, XGEN_DTYPE_BF16, N, diacc, stream));
  HIP_OK(hipStreamSynchronize(stream));
  host_copy(ix, dix, sizeof ix), host_copy(iw, diw, sizeof iw), host_copy(iacc, diacc, sizeof iacc);
  host_copy(sx, dsx, sizeof sx), host_copy(sw, dsw, sizeof sw), host_copy(out, dout, sizeof out);
  oracle_quant_rows_int8(XGEN_DTYPE_BF16, x, M, K, rix, rsx);
  oracle_quant_rows_int8(XGEN_DTYPE_BF16, w, N, K, riw, rsw);
  EXPECT(memcmp(ix, rix, sizeof ix) == 0 && memcmp(sx, rsx, sizeof sx) == 0, "int8 activation bytes / scales");
  EXPECT(memcmp(iw, riw, sizeof iw) == 0 && memcmp(sw, rsw, sizeof sw) == 0, "int8 weight bytes / scales");
  int bad_acc = 0, bad_out = 0;
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      int32_t sum = 0;
      for (int k = 0; k < K; ++k) sum += (int32_t)ix[m * K + k] * iw[n * K + k];
      bad_acc += sum != iacc[m * N + n];
      const float y = fmaf((float)sum, sx[m] * sw[n], bf16_value(bias[n]));
      if (fabsf(bf16_value(out[m * N + n]) - y) > ldexpf(fabsf(y), -8) + 1e-30f) ++bad_out;
    }
  EXPECT(bad_acc == 0, "int8 accumulators: %d differ from the integer sums", bad_acc);
  EXPECT(bad_out == 0, "int8 outputs: %d off the epilogue of the accumulators", bad_out);

  /* ---- indexed AdaLN modulation of the activations as [1, M, K] rows: bf16 after every step */
  enum { T = 3 };
  static uint16_t table[T * 2 * K], mod[M * K];
  static int64_t idx[M];
  for (int i = 0; i < T * 2 * K; ++i) table[i] = bf16_bits(bell() * 0.1f);
  for (int m = 0; m < M; ++m) idx[m] = (m * 7) % T;
  void *dtable = device_copy(table, sizeof table), *didx = device_copy(idx, sizeof idx);
  void *dmod = device_copy(NULL, sizeof mod);
  /* scale and shift are the two halves of each [2K] table row: row stride 2K */
  XGEN_OK_CALL(xgen_indexed_modulate(dx, (int64_t)M * K, K, (uint16_t *)dtable + K, 2 * K, dtable, 2 * K, T,
                                     didx, 1, M, K, 0, dmod, stream));
  HIP_OK(hipStreamSynchronize(stream));
  host_copy(mod, dmod, sizeof mod);
  int bad_mod = 0;
  for (int m = 0; m < M; ++m)
    for (int k = 0; k < K; ++k) {
      const uint16_t *row = table + idx[m] * 2 * K;
      const float f = bf16_value(bf16_bits(1.0f + bf16_value(row[K + k])));
      const float p = bf16_value(bf16_bits(bf16_value(x[m * K + k]) * f));
      bad_mod += mod[m * K + k] != bf16_bits(p + bf16_value(row[k]));
    }
  EXPECT(bad_mod == 0, "indexed modulation: %d values differ from the eager bf16 steps", bad_mod);

  /* ---- the error contract: checked before any launch, message per thread */
  EXPECT(xgen_quantize_rows(XGEN_DTYPE_BF16, dx, M, K, K, 42, dqx, K, dsx, stream) == XGEN_ERR_INVALID_ARGUMENT,
         "an unknown output dtype is rejected");
  EXPECT(strlen(xgen_last_error()) > 0, "the rejection leaves a message");
  EXPECT(xgen_scaled_mm_fp8(dqx, K, dqw, K, M, N, K, dsx, 1, dsw, 1, db, XGEN_DTYPE_BF16, XGEN_ACT_NONE, NULL,
                            XGEN_DTYPE_BF16, N, NULL, stream) == XGEN_ERR_INVALID_ARGUMENT,
         "a null output is rejected");

  void *bufs[] = {dx, dw, db, dqx, dqw, dsx, dsw, dacc, dout, dix, diw, diacc, dtable, didx, dmod};
  for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; ++i) HIP_OK(hipFree(bufs[i]));
  HIP_OK(hipStreamDestroy(stream));
  if (failures) {
    printf("%d check(s) failed\n", failures);
    return 1;
  }
  printf("c abi ok: fp8 and int8 quantizers and the modulation bit-exact, accumulators within bounds, "
         "M=%d N=%d K=%d\n", M, N, K);
  return 0;
}

/* capi_consumer.c -- a plain C caller of the library, through
 * include/zipserv.h and libzipserv.so only (no Python, no torch), in the
 * shape of the reference's own GEMM test (kernel_benchmark/test_mm.cu:
 * generate W and X, compress W on the host with InitBF16MatrixTripleBitmap,
 * copy the streams to the device, run BF16TripleBitmap_MM_API and
 * BF16TripleBitmap_Decompress_API, compare on the host).  The comparison is
 * against a host fp32 GEMM of the same bf16 operands (the reference compares
 * against cuBLAS and asserts nothing); decompress must return W bit for bit.
 * The same streams are then re-tiled on the device and the re-tiled GEMM and
 * decompress are checked the same way.  Prints one line and exits 0 when
 * every check passes, 1 otherwise. */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "zipserv.h"

#define CHECK_HIP(x)                                                                 \
  do {                                                                               \
    hipError_t e_ = (x);                                                             \
    if (e_ != hipSuccess) {                                                          \
      fprintf(stderr, "%s:%d: %s\n", __FILE__, __LINE__, hipGetErrorString(e_));     \
      exit(1);                                                                       \
    }                                                                                \
  } while (0)
#define CHECK_ZS(x)                                                                  \
  do {                                                                               \
    int s_ = (x);                                                                    \
    if (s_ != ZS_OK) {                                                               \
      fprintf(stderr, "%s:%d: %s -> %d (%s)\n", __FILE__, __LINE__, #x, s_,          \
              zs_status_string(s_));                                                 \
      exit(1);                                                                       \
    }                                                                                \
  } while (0)

static uint64_t lcg_state = 0x9E3779B97F4A7C15ull;
static double uniform01(void) {
  lcg_state = lcg_state * 6364136223846793005ull + 1442695040888963407ull;
  return (double)(lcg_state >> 11) / 9007199254740992.0;
}
/* roughly normal: sum of four uniforms, centred and scaled to unit variance */
static double normalish(void) {
  return (uniform01() + uniform01() + uniform01() + uniform01() - 2.0) * 1.7320508075688772;
}
static uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
static float bf16_to_f32(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static void* dev_copy(const void* host, size_t bytes, size_t capacity) {
  void* d = NULL;
  CHECK_HIP(hipMalloc(&d, capacity));
  CHECK_HIP(hipMemset(d, 0, capacity));
  if (bytes) CHECK_HIP(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice));
  return d;
}

/* max |y - ref| / max |ref| over an N x M output */
static double rel_err(const uint16_t* y, const float* ref, int64_t n) {
  double err = 0.0, scale = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const double d = fabs((double)bf16_to_f32(y[i]) - (double)ref[i]);
    if (d > err) err = d;
    if (fabs((double)ref[i]) > scale) scale = fabs((double)ref[i]);
  }
  return scale > 0.0 ? err / scale : err;
}

int main(void) {
  const int M = 512, K = 1024;
  const int Ns[3] = {1, 8, 40};
  int failures = 0;

  /* W: N(0, 0.02) bf16 with 0.5% of the entries x30 (outside the window) */
  uint16_t* W = (uint16_t*)malloc((size_t)M * K * 2);
  for (int64_t i = 0; i < (int64_t)M * K; ++i) {
    double v = 0.02 * normalish();
    if (uniform01() < 0.005) v *= 30.0;
    W[i] = f32_to_bf16((float)v);
  }

  /* host codec: window (utils.h:189-272) and the canonical streams */
  int32_t top[7];
  CHECK_ZS(zs_analyze_exponents_host(W, (int64_t)M * K, top));
  uint8_t* sm = NULL;
  uint16_t* full = NULL;
  uint64_t *b1 = NULL, *b2 = NULL, *b3 = NULL;
  int32_t *to = NULL, *tom = NULL, *tog = NULL;
  int32_t max_hf = 0, max_full = 0;
  const int ngt = zs_init_bf16_matrix_triple_bitmap(W, M, K, 8, 16, 64, 8, 64, 64, top, &sm,
                                                    &full, &b1, &b2, &b3, &to, &tom, &tog,
                                                    &max_hf, &max_full);
  if (ngt <= 0) {
    fprintf(stderr, "host encoder failed: %d\n", ngt);
    return 1;
  }
  const int64_t total_hf = tog[2 * ngt], total_full = tog[2 * ngt + 1];
  const uint8_t start_exp = (uint8_t)(top[0] - 1);
  const int64_t nsmall = (int64_t)M * K / 64, nmed = (int64_t)M * K / 1024;

  uint8_t* d_sm = (uint8_t*)dev_copy(sm, (size_t)total_hf, (size_t)zs_sign_mantissa_capacity(M, K));
  uint16_t* d_full = (uint16_t*)dev_copy(full, (size_t)total_full * 2,
                                         (size_t)zs_full_capacity(M, K) * 2);
  uint64_t* d_b1 = (uint64_t*)dev_copy(b1, (size_t)nsmall * 8, (size_t)nsmall * 8);
  uint64_t* d_b2 = (uint64_t*)dev_copy(b2, (size_t)nsmall * 8, (size_t)nsmall * 8);
  uint64_t* d_b3 = (uint64_t*)dev_copy(b3, (size_t)nsmall * 8, (size_t)nsmall * 8);
  int32_t* d_tom = (int32_t*)dev_copy(tom, (size_t)nmed * 2 * 4, (size_t)nmed * 2 * 4);
  int32_t* d_tog = (int32_t*)dev_copy(tog, (size_t)(ngt + 1) * 2 * 4, (size_t)(ngt + 1) * 2 * 4);

  /* decompress: W bit for bit */
  uint16_t* d_w = NULL;
  CHECK_HIP(hipMalloc((void**)&d_w, (size_t)M * K * 2));
  uint16_t* w_back = (uint16_t*)malloc((size_t)M * K * 2);
  CHECK_ZS(zs_bf16_triple_bitmap_decompress(NULL, d_sm, d_full, d_b1, d_b2, d_b3, d_tom, d_tog,
                                            max_hf, max_full, start_exp, d_w, M, K));
  CHECK_HIP(hipMemcpy(w_back, d_w, (size_t)M * K * 2, hipMemcpyDeviceToHost));
  if (memcmp(w_back, W, (size_t)M * K * 2) != 0) {
    fprintf(stderr, "canonical decompress differs from W\n");
    ++failures;
  }

  /* the same streams re-tiled on the device (two phases: sizes, then bytes) */
  const int64_t nrec = zs_retiled_num_records(M, K);
  int32_t *d_counts = NULL, *d_eoff = NULL;
  int64_t* d_total = NULL;
  CHECK_HIP(hipMalloc((void**)&d_counts, (size_t)nrec * 4));
  CHECK_HIP(hipMalloc((void**)&d_eoff, (size_t)(nrec + 1) * 4));
  CHECK_HIP(hipMalloc((void**)&d_total, 8));
  CHECK_ZS(zs_retile_triple_bitmap_count_gpu(NULL, d_sm, d_full, d_b1, d_b2, d_b3, d_tom, d_tog,
                                             M, K, d_counts, d_eoff, d_total));
  int64_t outliers = 0, expected = 0;
  CHECK_HIP(hipMemcpy(&outliers, d_total, 8, hipMemcpyDeviceToHost));
  /* one outlier byte per element outside the window top[0]..top[6] (the FULL
   * stream holds the same elements, padded to 8 per global tile) */
  for (int64_t i = 0; i < (int64_t)M * K; ++i) {
    const int e = (W[i] >> 7) & 0xFF;
    expected += e < top[0] || e > top[6];
  }
  if (outliers != expected || outliers > total_full) {
    fprintf(stderr, "re-tiled outlier count %lld, expected %lld (FULL, padded: %lld)\n",
            (long long)outliers, (long long)expected, (long long)total_full);
    ++failures;
  }
  uint8_t *d_fixed = NULL, *d_exps = NULL;
  CHECK_HIP(hipMalloc((void**)&d_fixed, (size_t)zs_retiled_fixed_bytes(M, K)));
  CHECK_HIP(hipMalloc((void**)&d_exps, (size_t)outliers + ZS_STREAM_SLACK_BYTES));
  CHECK_HIP(hipMemset(d_exps, 0, (size_t)outliers + ZS_STREAM_SLACK_BYTES));
  CHECK_ZS(zs_retile_triple_bitmap_emit_gpu(NULL, d_sm, d_full, d_b1, d_b2, d_b3, d_tom, d_tog,
                                            start_exp, M, K, d_eoff, d_fixed, d_exps));
  CHECK_HIP(hipMemset(d_w, 0, (size_t)M * K * 2));
  CHECK_ZS(zs_retiled_decompress(NULL, d_fixed, d_exps, d_eoff, start_exp, d_w, M, K));
  CHECK_HIP(hipMemcpy(w_back, d_w, (size_t)M * K * 2, hipMemcpyDeviceToHost));
  if (memcmp(w_back, W, (size_t)M * K * 2) != 0) {
    fprintf(stderr, "re-tiled decompress differs from W\n");
    ++failures;
  }

  /* ZipGEMM: C[N][M] = X[N][K] . W[M][K]^T, split-K 1 and 2, both layouts */
  for (int t = 0; t < 3; ++t) {
    const int N = Ns[t];
    uint16_t* X = (uint16_t*)malloc((size_t)N * K * 2);
    for (int64_t i = 0; i < (int64_t)N * K; ++i) X[i] = f32_to_bf16((float)normalish());
    float* ref = (float*)malloc((size_t)N * M * 4);
    for (int n = 0; n < N; ++n)
      for (int m = 0; m < M; ++m) {
        double acc = 0.0;
        for (int k = 0; k < K; ++k)
          acc += (double)bf16_to_f32(X[(int64_t)n * K + k]) * (double)bf16_to_f32(W[(int64_t)m * K + k]);
        ref[(int64_t)n * M + m] = (float)acc;
      }
    uint16_t* d_x = (uint16_t*)dev_copy(X, (size_t)N * K * 2, (size_t)N * K * 2);
    uint16_t *d_y = NULL, *d_ws = NULL;
    CHECK_HIP(hipMalloc((void**)&d_y, (size_t)N * M * 2));
    CHECK_HIP(hipMalloc((void**)&d_ws, (size_t)zs_splitk_workspace_bytes(M, N, 2)));
    uint16_t* y = (uint16_t*)malloc((size_t)N * M * 2);
    for (int split = 1; split <= 2; ++split) {
      for (int layout = 0; layout < 2; ++layout) {
        CHECK_HIP(hipMemset(d_y, 0xFF, (size_t)N * M * 2));
        if (layout == 0)
          CHECK_ZS(zs_bf16_triple_bitmap_mm(NULL, d_sm, d_full, d_b1, d_b2, d_b3, d_tom, d_tog,
                                            max_hf, max_full, start_exp, d_x, d_y, M, N, K, d_ws,
                                            split));
        else
          CHECK_ZS(zs_retiled_mm(NULL, d_fixed, d_exps, d_eoff, start_exp, d_x, d_y, M, N, K, d_ws,
                                 split));
        CHECK_HIP(hipDeviceSynchronize());
        CHECK_HIP(hipMemcpy(y, d_y, (size_t)N * M * 2, hipMemcpyDeviceToHost));
        const double e = rel_err(y, ref, (int64_t)N * M);
        if (!(e <= 1e-2)) {
          fprintf(stderr, "%s ZipGEMM N=%d split-K %d: relative error %g\n",
                  layout ? "re-tiled" : "canonical", N, split, e);
          ++failures;
        }
      }
    }
    /* unit vectors: X[n] = e_k gives Y[n] = W[:, k] exactly */
    for (int64_t i = 0; i < (int64_t)N * K; ++i) X[i] = 0;
    for (int n = 0; n < N; ++n) X[(int64_t)n * K + (n * 37 + 5) % K] = 0x3F80; /* 1.0 */
    CHECK_HIP(hipMemcpy(d_x, X, (size_t)N * K * 2, hipMemcpyHostToDevice));
    for (int layout = 0; layout < 2; ++layout) {
      if (layout == 0)
        CHECK_ZS(zs_bf16_triple_bitmap_mm(NULL, d_sm, d_full, d_b1, d_b2, d_b3, d_tom, d_tog,
                                          max_hf, max_full, start_exp, d_x, d_y, M, N, K, d_ws, 1));
      else
        CHECK_ZS(zs_retiled_mm(NULL, d_fixed, d_exps, d_eoff, start_exp, d_x, d_y, M, N, K, d_ws, 1));
      CHECK_HIP(hipMemcpy(y, d_y, (size_t)N * M * 2, hipMemcpyDeviceToHost));
      for (int n = 0; n < N; ++n) {
        const int k = (n * 37 + 5) % K;
        for (int m = 0; m < M; ++m) {
          /* compare as values (+0 == -0) */
          if (bf16_to_f32(y[(int64_t)n * M + m]) != bf16_to_f32(W[(int64_t)m * K + k])) {
            fprintf(stderr, "%s unit vector N=%d row %d column %d differs\n",
                    layout ? "re-tiled" : "canonical", N, n, m);
            ++failures;
            n = N;
            break;
          }
        }
      }
    }
    free(X);
    free(ref);
    free(y);
    CHECK_HIP(hipFree(d_x));
    CHECK_HIP(hipFree(d_y));
    CHECK_HIP(hipFree(d_ws));
  }

  /* arguments the reference does not validate are refused here */
  if (zs_bf16_triple_bitmap_mm(NULL, d_sm, d_full, d_b1, d_b2, d_b3, d_tom, d_tog, max_hf,
                               max_full, start_exp, NULL, NULL, M, 8, K, NULL, 1) != ZS_E_INVAL) {
    fprintf(stderr, "null operands were not refused\n");
    ++failures;
  }

  zs_host_free(sm);
  zs_host_free(full);
  zs_host_free(b1);
  zs_host_free(b2);
  zs_host_free(b3);
  zs_host_free(to);
  zs_host_free(tom);
  zs_host_free(tog);
  free(W);
  free(w_back);
  void* dev[] = {d_sm, d_full, d_b1, d_b2, d_b3, d_tom, d_tog, d_w, d_counts, d_eoff, d_total,
                 d_fixed, d_exps};
  for (size_t i = 0; i < sizeof(dev) / sizeof(dev[0]); ++i) CHECK_HIP(hipFree(dev[i]));
  if (failures) {
    printf("capi_consumer: %d check(s) failed\n", failures);
    return 1;
  }
  printf("capi_consumer: ok (M=%d K=%d, N=1/8/40, split-K 1/2, canonical and re-tiled, "
         "ratio %.4f)\n",
         M, K, 2.0 * M * K / (double)zs_compressed_bytes(M, K, total_hf, total_full));
  return 0;
}

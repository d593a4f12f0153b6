/*
 * A C99 host program of libkda.so: the C ABI of include/kda.h used from C with
 * the HIP runtime's C API, no C++ and no Python.
 *
 *   silu_host --validate   calls that fail argument validation (no GPU is touched):
 *                          the status codes and kda_last_error() messages
 *   silu_host [n]          y = silu(x) on the GPU for n fp32 values in [-12, 12)
 *                          (default 2^20 + 3: the vector kernel and the scalar tail),
 *                          checked against x / (1 + exp(-x)) evaluated in double on the
 *                          host: every element within 4e-6 relative (the kernel's exp
 *                          is exp2(x * log2(e)) in fp32, whose rounded argument alone
 *                          moves exp(-12) by up to about 1.3e-6 relative)
 *
 * Exit status 0 when every check passes.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "kda.h"

static int validate(void) {
  int fails = 0;
  if (kda_version() != 100) {
    fprintf(stderr, "version %d\n", kda_version());
    ++fails;
  }
  int rc = kda_silu_f32(NULL, NULL, -1, NULL);
  printf("silu n=-1: rc=%d msg='%s'\n", rc, kda_last_error());
  if (rc != KDA_ERR_INVALID_ARG || strstr(kda_last_error(), "n=-1") == NULL) ++fails;
  rc = kda_silu_f32(NULL, NULL, 16, NULL);
  printf("silu null: rc=%d msg='%s'\n", rc, kda_last_error());
  if (rc != KDA_ERR_INVALID_ARG || strstr(kda_last_error(), "null pointer") == NULL) ++fails;
  rc = kda_silu_f32(NULL, NULL, 0, NULL);   /* nothing to do: succeeds, clears the message */
  printf("silu n=0: rc=%d msg='%s'\n", rc, kda_last_error());
  if (rc != KDA_OK || kda_last_error()[0] != '\0') ++fails;
  return fails;
}

#define HIP_OK(call)                                                     \
  do {                                                                   \
    hipError_t e_ = (call);                                              \
    if (e_ != hipSuccess) {                                              \
      fprintf(stderr, "%s: %s\n", #call, hipGetErrorString(e_));         \
      return 2;                                                          \
    }                                                                    \
  } while (0)

static int run(int64_t n) {
  float* x = (float*)malloc((size_t)n * sizeof(float));
  float* y = (float*)malloc((size_t)n * sizeof(float));
  if (!x || !y) return 2;
  uint32_t s = 12345u;
  for (int64_t i = 0; i < n; ++i) {   /* values in [-12, 12) from a 32-bit LCG */
    s = s * 1664525u + 1013904223u;
    x[i] = (float)((double)(s >> 8) / (double)(1u << 24) * 24.0 - 12.0);
  }
  float *dx = NULL, *dy = NULL;
  HIP_OK(hipMalloc((void**)&dx, (size_t)n * sizeof(float)));
  HIP_OK(hipMalloc((void**)&dy, (size_t)n * sizeof(float)));
  HIP_OK(hipMemcpy(dx, x, (size_t)n * sizeof(float), hipMemcpyHostToDevice));
  hipStream_t stream;
  HIP_OK(hipStreamCreate(&stream));
  const int rc = kda_silu_f32(dx, dy, n, (void*)stream);
  if (rc != KDA_OK) {
    fprintf(stderr, "kda_silu_f32: rc=%d %s\n", rc, kda_last_error());
    return 1;
  }
  HIP_OK(hipStreamSynchronize(stream));
  HIP_OK(hipMemcpy(y, dy, (size_t)n * sizeof(float), hipMemcpyDeviceToHost));
  double worst = 0.0;
  int64_t at = 0;
  for (int64_t i = 0; i < n; ++i) {
    const double want = (double)x[i] / (1.0 + exp(-(double)x[i]));
    const double err = fabs((double)y[i] - want) / (fabs(want) + 1e-30);
    if (!(err <= worst)) {   /* also catches NaN */
      worst = err;
      at = i;
    }
  }
  printf("silu n=%lld: worst relative error %.3e at %lld (x=%.9g y=%.9g)\n", (long long)n, worst,
         (long long)at, x[at], y[at]);
  HIP_OK(hipStreamDestroy(stream));
  HIP_OK(hipFree(dx));
  HIP_OK(hipFree(dy));
  free(x);
  free(y);
  return worst < 4e-6 ? 0 : 1;
}

int main(int argc, char** argv) {
  if (argc > 1 && strcmp(argv[1], "--validate") == 0) return validate();
  const int64_t n = argc > 1 ? atoll(argv[1]) : (int64_t)(1 << 20) + 3;
  if (n <= 0) return 2;
  return run(n);
}

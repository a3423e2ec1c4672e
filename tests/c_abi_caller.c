/*
 * A plain C caller of libfqkv_decode.so: no Python, no PyTorch. It allocates
 * device memory with the HIP runtime, runs fqkv_gqa_sk_fast and
 * fqkv_decode_attn_gqa (GQA, Hq 32 / Hkv 8, D 128) on fp16 data made here, and
 * checks both against a double-precision softmax(q K^T / sqrt(D)) V computed
 * on the host from the same fp16 values. Prints "OK <max-abs error>" and
 * exits 0 when both are within 2e-3, non-zero otherwise.
 *
 * Built by tests/test_gpu_cabi.py with gcc against include/fqkv_decode.h.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "fqkv_decode.h"

/* IEEE binary32 -> binary16, round to nearest even (finite inputs of modest size). */
static uint16_t f2h(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const int32_t e = (int32_t)((x >> 23) & 0xffu) - 127 + 15;
  uint32_t mant = x & 0x7fffffu;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    mant |= 0x800000u;
    const int shift = 14 - e;
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return (uint16_t)(sign | h);
}

static double h2d(uint16_t h) {
  const int e = (h >> 10) & 0x1f, m = h & 0x3ff;
  const double s = (h & 0x8000) ? -1.0 : 1.0;
  if (e == 0) return s * ldexp((double)m, -24);
  return s * ldexp((double)(m | 0x400), e - 25);
}

static uint32_t rng = 12345u;
static float uniform(void) { /* [-2, 2) */
  rng = rng * 1664525u + 1013904223u;
  return (float)(rng >> 8) / (float)(1u << 24) * 4.0f - 2.0f;
}

#define CHECK_HIP(x)                                                       \
  do {                                                                     \
    hipError_t e_ = (x);                                                   \
    if (e_ != hipSuccess) {                                                \
      fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));      \
      return 2;                                                            \
    }                                                                      \
  } while (0)
#define CHECK_FQKV(x)                                                      \
  do {                                                                     \
    if ((x) != FQKV_OK) {                                                  \
      fprintf(stderr, "%s failed: %s\n", #x, fqkv_last_error());          \
      return 3;                                                            \
    }                                                                      \
  } while (0)

int main(void) {
  const int64_t Hq = 32, Hkv = 8, N = 1000, D = 128, S = 16, G = Hq / Hkv;
  const size_t nq = (size_t)(Hq * D), nkv = (size_t)(Hkv * N * D);
  uint16_t* q = malloc(nq * 2);
  uint16_t* K = malloc(nkv * 2);
  uint16_t* V = malloc(nkv * 2);
  uint16_t* o = malloc(nq * 2);
  double* ref = malloc(nq * sizeof(double));
  double* p = malloc((size_t)N * sizeof(double));
  if (!q || !K || !V || !o || !ref || !p) return 4;
  for (size_t i = 0; i < nq; ++i) q[i] = f2h(uniform());
  for (size_t i = 0; i < nkv; ++i) K[i] = f2h(uniform());
  for (size_t i = 0; i < nkv; ++i) V[i] = f2h(uniform());

  /* host reference: head h reads KV head h / G */
  for (int64_t h = 0; h < Hq; ++h) {
    const uint16_t* kh = K + (size_t)(h / G) * N * D;
    const uint16_t* vh = V + (size_t)(h / G) * N * D;
    double mx = -INFINITY, l = 0.0;
    for (int64_t t = 0; t < N; ++t) {
      double s = 0.0;
      for (int64_t d = 0; d < D; ++d) s += h2d(q[h * D + d]) * h2d(kh[t * D + d]);
      p[t] = s / sqrt((double)D);
      if (p[t] > mx) mx = p[t];
    }
    for (int64_t t = 0; t < N; ++t) l += (p[t] = exp(p[t] - mx));
    for (int64_t d = 0; d < D; ++d) {
      double acc = 0.0;
      for (int64_t t = 0; t < N; ++t) acc += p[t] * h2d(vh[t * D + d]);
      ref[h * D + d] = acc / l;
    }
  }

  void *dq, *dK, *dV, *dO, *dM, *dL, *dOp, *dW = NULL;
  CHECK_HIP(hipMalloc(&dq, nq * 2));
  CHECK_HIP(hipMalloc(&dK, nkv * 2));
  CHECK_HIP(hipMalloc(&dV, nkv * 2));
  CHECK_HIP(hipMalloc(&dO, nq * 2));
  CHECK_HIP(hipMalloc(&dM, (size_t)(Hq * S) * 4));
  CHECK_HIP(hipMalloc(&dL, (size_t)(Hq * S) * 4));
  CHECK_HIP(hipMalloc(&dOp, (size_t)(Hq * S * D) * 4));
  CHECK_HIP(hipMemcpy(dq, q, nq * 2, hipMemcpyHostToDevice));
  CHECK_HIP(hipMemcpy(dK, K, nkv * 2, hipMemcpyHostToDevice));
  CHECK_HIP(hipMemcpy(dV, V, nkv * 2, hipMemcpyHostToDevice));

  double worst = 0.0;
  for (int call = 0; call < 2; ++call) {
    CHECK_HIP(hipMemset(dO, 0, nq * 2));
    if (call == 0) {
      CHECK_FQKV(fqkv_gqa_sk_fast(dq, dK, dV, (float*)dM, (float*)dL, (float*)dOp, dO, Hq, Hkv, N, D, S, 8, 8,
                                  NULL));
    } else {
      const size_t ws = fqkv_workspace_bytes(Hkv, G, N, D, FQKV_KV_F16, 8);
      if (ws) CHECK_HIP(hipMalloc(&dW, ws));
      CHECK_FQKV(fqkv_decode_attn_gqa(dq, dK, dV, dO, 1, Hq, Hkv, N, D, 8, dW, ws, NULL));
    }
    CHECK_HIP(hipDeviceSynchronize());
    CHECK_HIP(hipMemcpy(o, dO, nq * 2, hipMemcpyDeviceToHost));
    double err = 0.0;
    for (size_t i = 0; i < nq; ++i) {
      const double e = fabs(h2d(o[i]) - ref[i]);
      if (!(e <= err)) err = e; /* NaN propagates */
    }
    printf("%s max-abs error %.3e\n", call == 0 ? "fqkv_gqa_sk_fast" : "fqkv_decode_attn_gqa", err);
    if (!(err <= worst)) worst = err;
  }
  hipFree(dq);
  hipFree(dK);
  hipFree(dV);
  hipFree(dO);
  hipFree(dM);
  hipFree(dL);
  hipFree(dOp);
  if (dW) hipFree(dW);
  free(q);
  free(K);
  free(V);
  free(o);
  free(ref);
  free(p);
  if (!(worst <= 2e-3)) {
    printf("FAIL %.3e\n", worst);
    return 1;
  }
  printf("OK %.3e\n", worst);
  return 0;
}

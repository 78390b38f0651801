/*
 * CPU oracle / CPU baseline: fp32 GEMM in the loop order of the reference's
 * native CPU tier. TEST INFRASTRUCTURE ONLY (never linked into the product).
 *
 * zko_matmul_f32_avx2 follows matmul_f32_avx2 (core/src/cpu_kernels.cpp:
 * 129-165): C is zeroed, then for every row i and every k the scalar A[i,k]
 * is broadcast and multiplied into row k of B eight columns at a time with
 * one fused multiply-add, C being re-loaded and re-stored on every k; the
 * column tail is scalar. Single-threaded, as in the reference.
 * zko_matmul_f32_naive follows matmul_f32_naive (cpu_kernels.cpp:108-122).
 */
#include <immintrin.h>
#include <stddef.h>
#include <string.h>

void zko_matmul_f32_naive(const float *A, const float *B, float *C, int M,
                          int N, int K) {
  memset(C, 0, sizeof(float) * (size_t)M * (size_t)N);
  for (int i = 0; i < M; ++i)
    for (int k = 0; k < K; ++k) {
      const float a = A[(size_t)i * K + k];
      for (int j = 0; j < N; ++j) C[(size_t)i * N + j] += a * B[(size_t)k * N + j];
    }
}

void zko_matmul_f32_avx2(const float *A, const float *B, float *C, int M,
                         int N, int K) {
  memset(C, 0, sizeof(float) * (size_t)M * (size_t)N);
  const int n8 = N - N % 8;
  for (int i = 0; i < M; ++i) {
    float *crow = C + (size_t)i * N;
    for (int k = 0; k < K; ++k) {
      const float a = A[(size_t)i * K + k];
      const float *brow = B + (size_t)k * N;
      const __m256 av = _mm256_set1_ps(a);
      int j = 0;
      for (; j < n8; j += 8) {
        __m256 c = _mm256_loadu_ps(crow + j);
        c = _mm256_fmadd_ps(av, _mm256_loadu_ps(brow + j), c);
        _mm256_storeu_ps(crow + j, c);
      }
      for (; j < N; ++j) crow[j] += a * brow[j];
    }
  }
}

// Shared definitions for the gfx950 kernels of libzenith_hip.so:
// vector types, MFMA wrappers, wave reductions, argument checking and the
// thread-local last-error slot behind zk_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/zk_api.h"

namespace zk {

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- errors --
// Set the thread-local error text; returns `code` so callers can
// `return fail(ZK_ERR_INVALID, "...")`.
int fail(int code, const char *fmt, ...);
// Check hipGetLastError() after a launch.
int check_launch(const char *what);
// 16-byte alignment of a device pointer.
__host__ __device__ inline bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}
inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------ device math --
__device__ __forceinline__ float gelu_erf(float x) {
  // 0.5 x (1 + erf(x / sqrt(2)))
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
}
__device__ __forceinline__ float gelu_tanh(float x) {
  // 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), Hendrycks & Gimpel
  const float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

// Branch-free forms for GEMM epilogues (fp16 outputs).
// erf by Abramowitz & Stegun 7.1.26: for z >= 0,
//   erf(z) = 1 - (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) exp(-z^2),
//   t = 1 / (1 + p z), |error| <= 1.5e-7.
__device__ __forceinline__ float gelu_erf_fast(float x) {
  const float z = fabsf(x) * 0.70710678118654752f;
  const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * z);
  float q = 1.061405429f;
  q = q * t - 1.453152027f;
  q = q * t + 1.421413741f;
  q = q * t - 0.284496736f;
  q = q * t + 0.254829592f;
  q *= t;
  // 1 - erf(z), then GELU = 0.5 x (1 + sign(x) erf(|x| / sqrt 2))
  const float tail = q * __builtin_amdgcn_exp2f(-z * z * 1.4426950408889634f);
  return x >= 0.f ? x - 0.5f * x * tail : 0.5f * x * tail;
}
// tanh(y) = 1 - 2 / (1 + exp(2y)): exact identity, one exp and one reciprocal.
__device__ __forceinline__ float gelu_tanh_fast(float x) {
  const float y = 0.7978845608028654f * (x + 0.044715f * x * x * x);
  const float e = __builtin_amdgcn_exp2f(2.0f * 1.4426950408889634f * y);
  const float th = 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + e);
  return 0.5f * x * (1.0f + th);
}

// Butterfly sum / max across the 64 lanes of a wavefront.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// ------------------------------------------------------------------ MFMA --
// D(32x32, fp32) += A(32x16, f16) . B(16x32, f16). Lane l supplies
// A[l%32][8*(l/32) .. +7] and B[8*(l/32) .. +7][l%32]; it receives
// D[8*(r/4) + 4*(l/32) + r%4][l%32] in register r.
__device__ __forceinline__ f32x16 mfma32x32x16(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
// Same shape for int8 with K = 32 (16 bytes per lane and operand).
__device__ __forceinline__ i32x16 mfma32x32x32_i8(i32x4 a, i32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

}  // namespace zk

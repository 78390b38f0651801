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

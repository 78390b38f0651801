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
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Output stores are non-temporal (streaming): the written lines are not
// kept in the writer's cache, which measured faster for every producer
// here whose result is read by the next kernel (it is still served from
// the memory-side cache) and for results written once.
template <typename V>
__device__ __forceinline__ void store_nt(V *p, V v) {
  __builtin_nontemporal_store(v, p);
}

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
__host__ __device__ inline bool aligned8(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 7u) == 0;
}
inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// The fp16 GEMM behind zk_gemm_f16 / zk_gemm_f16_ws (zk_gemm.hip): with a
// device workspace `ws` of at least zk_gemm_workspace_size bytes, small-M
// products are split along K through it; with none they run unsplit.
int gemm_f16_impl(const void *A, const void *B, void *C, int64_t M, int64_t N, int64_t K,
                  int64_t lda, int64_t ldb, int64_t ldc, int trans_b, int out_dtype,
                  const void *bias, const void *residual, int64_t ldr, int epilogue, void *ws,
                  int64_t ws_bytes, void *stream);

// Add+LayerNorm over split-K partials (zk_layernorm.hip): y = LN(x + res)
// with x = fp16(sum of the `splits` fp32 partials [rows][hidden], split s at
// ws + s * stride, + bias), the same values and the same LayerNorm as
// splitk_reduce (ZK_EPI_BIAS) followed by zk_layernorm. ln_partials_ok says
// whether the shape and alignments allow it (hidden a multiple of 8 up to
// 8192, 16-byte aligned operands).
// With `wide` (allowed when ln_partials_wide_ok) each row gets a workgroup
// of four wavefronts to form it from the partials.
bool ln_partials_ok(const float *ws, int64_t stride, const void *bias, const void *res,
                    const void *g, const void *b, const void *y, int64_t rows, int64_t hidden);
bool ln_partials_wide_ok(int64_t rows, int64_t hidden);
int ln_add_partials_f16(const float *ws, int splits, int64_t stride, const void *bias,
                        const void *res, const void *g, const void *b, void *y, int64_t rows,
                        int64_t hidden, float eps, bool wide, hipStream_t s);

// Symmetric int8 quantisation of one value,
//   q = clamp(round_half_even(RN(x / scale)), -128, 127)
// (quantize_f32_to_int8_kernel, core/src/cuda_kernels.cu:926-927), with
// inv = RN(1 / scale) computed once by the caller. t = RN(x * inv) is within
// 3 * 2^-24 |x / scale| of RN(x / scale) (three roundings of at most 2^-24
// each), i.e. within 2.4e-5 for |t| < 129, so rint(t) is the exact answer
// unless t lies within 6e-5 of a half-integer; those values (about one in
// ten thousand) take the IEEE division (hipcc keeps fp32 '/' correctly
// rounded). For |t| >= 129 both forms saturate, whichever path is taken.
// NaN gives 0, as in the reference: its kernel rounds with a float-to-int
// conversion that turns NaN into 0 before the clamp, and its numpy rule
// (benchmarks/int8_bench.py:24) casts the NaN left by np.clip to 0 on x86.
__device__ __forceinline__ int8_t quant1(float x, float scale, float inv) {
  const float t = x * inv;
  float r = __builtin_rintf(t);
  if (fabsf(t - r) >= 0.49994f) r = __builtin_rintf(x / scale);
  r = fminf(fmaxf(r, -128.0f), 127.0f);
  return x != x ? (int8_t)0 : (int8_t)(int)r;
}

// Eight values at once, the same result as quant1 on each, packed as int8.
// t = RN(x * inv + 128) is one rounding of the exact x * inv + 128, so for
// |x / scale| <= 128.5 it lies within 1.6e-5 + 7.7e-6 of x / scale + 128,
// and within 3.1e-5 of RN(x / scale) + 128; rint(t) - 128 is therefore the
// exact answer unless t lies within 6e-5 of a half-integer, and the group
// takes the IEEE division when any of its eight does. Beyond 128.5 both
// forms saturate. The offset makes every clamped value a byte in [0, 255]:
// packed by v_cvt_pk_u8_f32 (exact on integers), then shifted back to
// int8 by flipping each byte's top bit. The clamp is v_med3_f32, which
// returns the minimum (0) when an operand is NaN, so a NaN must not reach
// it: the sum of the eight t is NaN when one of them is (or when +inf and
// -inf meet), and such a group takes the careful path too, where a NaN
// becomes the byte 128, i.e. 0 as in quant1.
__device__ __forceinline__ u32x2 quant8(const float (&x)[8], float scale, float inv) {
  float r[8], dev = 0.f, sum = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float t = fmaf(x[e], inv, 128.0f);
    r[e] = __builtin_rintf(t);
    dev = fmaxf(dev, fabsf(t - r[e]));
    sum += t;
  }
  if (dev >= 0.49994f || sum != sum) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      r[e] = x[e] != x[e] ? 128.0f : __builtin_rintf(x[e] / scale) + 128.0f;
  }
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    lo = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_amdgcn_fmed3f(r[e], 0.f, 255.f), e, lo);
    hi = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_amdgcn_fmed3f(r[e + 4], 0.f, 255.f), e, hi);
  }
  return u32x2{lo ^ 0x80808080u, hi ^ 0x80808080u};
}

// ------------------------------------------------------------ split-K sums --
// The sum over splits 0 .. splits-1 of the value at p + split * stride
// (float or f32x4), added in split order starting from zero, as a loop of
// one load and one add per split would; the loads are issued eight at a time
// (past the last split, split s0's value is loaded again and not added), so
// that a thread waits for memory once per eight splits instead of per split.
template <typename V>
__device__ __forceinline__ V sum_splits(const float *p, int splits, int64_t stride) {
  V t = {};
  for (int s0 = 0; s0 < splits; s0 += 8) {
    V q[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      q[u] = *(const V *)(p + (int64_t)(s0 + u < splits ? s0 + u : s0) * stride);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (s0 + u < splits) t += q[u];
  }
  return t;
}

// ------------------------------------------------------------ device math --
// x as an fp32 value in a register: the compiler may otherwise fuse the fma
// that produced it with a following conversion to fp16 (v_fma_mix*_f16,
// one rounding where the source has two, to fp32 and then to fp16), and
// whether it does depends on the surrounding code, so two kernels with the
// same arithmetic could round a few values differently.
__device__ __forceinline__ float as_f32(float x) {
  asm volatile("" : "+v"(x));
  return x;
}
__device__ __forceinline__ float gelu_erf(float x) {
  // 0.5 x (1 + erf(x / sqrt(2)))
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
}
__device__ __forceinline__ float gelu_tanh(float x) {
  // 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), Hendrycks & Gimpel
  const float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

// Branch-free forms for GEMM epilogues (fp16 outputs), with the constant
// factors folded so that each costs as few VALU instructions as possible.
// erf-GELU: GELU(x) = x Phi(x) = max(x, 0) - |x| Phi(-|x|) for either sign
// (Phi the standard normal CDF), and Phi(-a) = 2^p(a) with p a degree-5
// polynomial, p(0) = -1 exactly (Phi(0) = 1/2), fitted to log2 Phi(-a) on
// [0, 8] by weighted minimax: a linear program over 4000 Chebyshev points
// with weight a Phi(-a) ln 2, the absolute error of the product per unit
// error in p (fit_gelu_poly.py beside this file prints the coefficients).
// The leading coefficient is negative and p falls monotonically beyond the
// fitted range (p < -52 for every a > 8), so 2^p underflows to 0 and
// GELU(x) = max(x, 0) there without a clamp. Evaluated in fp32 (Horner with
// fma, v_exp_f32): at most 7.2e-7 absolute against the exact GELU on
// [-12, 12] (the fp32 rounding of the result alone is up to 2.4e-7), and
// 6e-6 relative for 0 < |x| <= 1. Eight instructions, one of them
// transcendental (quarter rate, so it costs four).
__device__ __forceinline__ float gelu_erf_fast(float x) {
  const float a = fabsf(x);
  float p = -4.891129793e-04f;
  p = fmaf(p, a, 7.206471637e-03f);
  p = fmaf(p, a, -5.216677114e-02f);
  p = fmaf(p, a, -4.595749378e-01f);
  p = fmaf(p, a, -1.151007652e+00f);
  p = fmaf(p, a, -1.0f);
  return fmaf(-a, __builtin_amdgcn_exp2f(p), fmaxf(x, 0.f));
}
// tanh(y) = 1 - 2 / (1 + exp(2y)) (exact identity), so
// 0.5 x (1 + tanh(y)) = x - x / (1 + exp(2y)), y = sqrt(2/pi) (x + 0.044715 x^3).
__device__ __forceinline__ float gelu_tanh_fast(float x) {
  constexpr float c1 = 2.0f * 1.4426950408889634f * 0.7978845608028654f;
  constexpr float c3 = c1 * 0.044715f;
  const float e = __builtin_amdgcn_exp2f(x * fmaf(c3, x * x, c1));
  return fmaf(-x, __builtin_amdgcn_rcpf(1.0f + e), x);
}

// One butterfly step without the LDS: op(t, t of lane l ^ O), op commutative
// (a sum or a max: the order of its operands does not change the result).
// - O = 32, 16: v_permlane32_swap / v_permlane16_swap, whose two results hold
//   the pair {t(l), t(l ^ O)} in one order or the other;
// - O = 8, 4: a DPP rotation of each 16-lane row by O, which pairs lane l with
//   l ^ O wherever t repeats with period 2 O along the row: always for 8, and
//   for 4 once the step with offset 8 has been done;
// - O = 2, 1: a DPP permutation within each group of four lanes (exact).
template <int O, typename Op>
__device__ __forceinline__ float bfly(float t, Op op) {
  static_assert(O == 32 || O == 16 || O == 8 || O == 4 || O == 2 || O == 1, "butterfly offset");
  if constexpr (O == 32 || O == 16) {
    const unsigned u = __float_as_uint(t);
    const auto r = O == 32 ? __builtin_amdgcn_permlane32_swap(u, u, false, false)
                           : __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  } else {
    // row_ror:O, or quad_perm [1, 0, 3, 2] (O = 1) / [2, 3, 0, 1] (O = 2)
    constexpr int ctrl = O >= 4 ? 0x120 + O : (O == 1 ? 0xB1 : 0x4E);
    const float q =
        __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t), ctrl, 0xF, 0xF, false));
    return op(t, q);
  }
}
// t of lane l ^ 1 (a DPP quad permutation, exact)
__device__ __forceinline__ float lane_xor1(float t) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t), 0xB1, 0xF, 0xF, false));
}
struct OpAdd {
  __device__ float operator()(float a, float b) const { return a + b; }
};
struct OpMax {
  __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
// op over the N lanes of each aligned group of N (N = 2, 4, 16, 32 or 64),
// the same pairing and order as a loop of __shfl_xor from N / 2 down to 1
template <int N, typename Op>
__device__ __forceinline__ float group_reduce(float t, Op op) {
  static_assert(N == 64 || N == 32 || N == 16 || N == 4 || N == 2, "group size");
  if constexpr (N >= 64) t = bfly<32>(t, op);
  if constexpr (N >= 32) t = bfly<16>(t, op);
  if constexpr (N >= 16) t = bfly<8>(t, op);
  if constexpr (N >= 8) t = bfly<4>(t, op);
  if constexpr (N >= 4) t = bfly<2>(t, op);
  if constexpr (N >= 2) t = bfly<1>(t, op);
  return t;
}

// Butterfly sum / max across the 64 lanes of a wavefront.
__device__ __forceinline__ float wave_sum(float v) { return group_reduce<64>(v, OpAdd{}); }
__device__ __forceinline__ float wave_max(float v) { return group_reduce<64>(v, OpMax{}); }

// ------------------------------------------------------------ LDS DMA --
// Buffer loads that write LDS directly (buffer_load ... lds) are counted by
// vmcnt like any load. A ring of stages is consumed as: wait until the
// stage about to be read has landed (leaving younger stages in flight),
// then meet at lds_barrier.
#define ZK_LDS(p) ((__attribute__((address_space(3))) void *)(p))

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Wait until at most min(allowed, N) slices of PER instructions each, plus
// EXTRA loads issued after them, are still in flight (allowed is
// wave-uniform).
template <int N, int PER, int EXTRA = 0>
__device__ __forceinline__ void wait_slices(int allowed) {
  if constexpr (N == 0) {
    wait_vmcnt<EXTRA>();
  } else {
    if (allowed >= N) wait_vmcnt<N * PER + EXTRA>();
    else wait_slices<N - 1, PER, EXTRA>(allowed);
  }
}
// Workgroup barrier without the fence __syncthreads() carries: the fence
// would make the compiler wait for every outstanding LDS DMA, including the
// slices deliberately left in flight. Completion of the slice about to be
// read is established by the explicit vmcnt wait before it.
// The wave's own outstanding LDS reads are completed first, so that a
// stage every wave has issued its last reads of is safe to refill after it.
// (The wait is the compiler-visible builtin, simm16 0xC07F = lgkmcnt(0)
// with vmcnt and expcnt left open, so the compiler knows those fragment
// registers are ready and adds no later wait on younger reads.)
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
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

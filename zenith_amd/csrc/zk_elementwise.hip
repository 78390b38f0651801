// Bandwidth-bound elementwise kernels: ReLU, sigmoid, tanh, (bias+)GELU, int8 quantisation
// and the fp16 transpose. Every kernel moves 16-byte vectors per lane where
// the shape and alignment allow it and falls back to a scalar grid-stride
// loop otherwise.
#include <type_traits>

#include "zk_common.hpp"

namespace zk {

template <typename T> struct Vec16;
template <> struct Vec16<f16> { typedef f16x8 type; static constexpr int n = 8; };
template <> struct Vec16<float> { typedef f32x4 type; static constexpr int n = 4; };

static inline int grid_for(int64_t work, int block) {
  int64_t g = (work + block - 1) / block;
  if (g > 65536) g = 65536;  // grid-stride loops cover the rest
  if (g < 1) g = 1;
  return (int)g;
}

// ---------------------------------------------- ReLU, sigmoid, tanh --
// One grid-stride kernel per op over 16-byte vectors, then a scalar tail.
// fp16 values are computed in fp32 and rounded once. sigmoid is
// 1 / (1 + expf(-x)) with the IEEE division (0 for x below about -88, 1
// above about 17); tanh is the device library's tanhf.
enum UnaryOp { kRelu = 0, kSigmoid = 1, kTanh = 2 };

template <int OP>
__device__ inline float unary(float v) {
  if constexpr (OP == kRelu) return v > 0.f ? v : 0.f;
  else if constexpr (OP == kSigmoid) return 1.0f / (1.0f + expf(-v));
  else return tanhf(v);
}

template <int OP, typename T>
__global__ void unary_vec(const T *__restrict__ x, T *__restrict__ y,
                          int64_t nvec) {
  typedef typename Vec16<T>::type V;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nvec;
       i += stride) {
    V v = reinterpret_cast<const V *>(x)[i];
#pragma unroll
    for (int j = 0; j < Vec16<T>::n; ++j) v[j] = (T)unary<OP>((float)v[j]);
    store_nt(reinterpret_cast<V *>(y) + i, v);
  }
}

template <int OP, typename T>
__global__ void unary_scalar(const T *__restrict__ x, T *__restrict__ y,
                             int64_t begin, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = begin + blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
       i < n; i += stride)
    y[i] = (T)unary<OP>((float)x[i]);
}

template <int OP, typename T>
static int unary_impl(const void *xv, void *yv, int64_t n, hipStream_t s,
                      const char *name) {
  const T *x = (const T *)xv;
  T *y = (T *)yv;
  constexpr int W = Vec16<T>::n;
  int64_t nvec = (aligned16(x) && aligned16(y)) ? n / W : 0;
  if (nvec > 0) unary_vec<OP, T><<<grid_for(nvec, 256), 256, 0, s>>>(x, y, nvec);
  if (nvec * W < n)
    unary_scalar<OP, T><<<grid_for(n - nvec * W, 256), 256, 0, s>>>(x, y, nvec * W, n);
  return check_launch(name);
}

template <int OP>
static int unary_entry(const void *x, void *y, int64_t n, int dtype, void *stream,
                       const char *name) {
  if (n < 0) return fail(ZK_ERR_INVALID, "%s: negative size", name);
  if (n == 0) return ZK_OK;
  if (!x || !y) return fail(ZK_ERR_INVALID, "%s: null pointer", name);
  if (dtype == ZK_F32) return unary_impl<OP, float>(x, y, n, as_stream(stream), name);
  if (dtype == ZK_F16) return unary_impl<OP, f16>(x, y, n, as_stream(stream), name);
  return fail(ZK_ERR_UNSUPPORTED, "%s: dtype %d not supported", name, dtype);
}

// ------------------------------------------------------------------ GELU --
// fp16 outputs use the branch-free forms of the GEMM epilogues (GELU within
// 7.2e-7 absolute, far below fp16's 4.9e-4 relative step), so the kernel stays
// bound by HBM rather than by libm's erff / tanhf; fp32 keeps the exact forms.
template <typename T, int MODE>
__device__ __forceinline__ float gelu(float v) {
  if constexpr (std::is_same<T, f16>::value)
    return MODE == ZK_GELU_ERF ? gelu_erf_fast(v) : gelu_tanh_fast(v);
  else
    return MODE == ZK_GELU_ERF ? gelu_erf(v) : gelu_tanh(v);
}

// Row-blocked form for cols % W == 0: a thread owns one 16-byte column
// vector (its bias slice is loaded once) and handles kGeluRows rows per pass,
// issuing all of their loads before any arithmetic, so that each wavefront
// keeps kGeluRows KB in flight.
constexpr int kGeluRows = 4;
constexpr int kGeluBlock = 128;

template <typename T, int MODE, bool BIAS>
__global__ __launch_bounds__(kGeluBlock) void gelu_rows(const T *__restrict__ x,
                                                       const T *__restrict__ bias,
                                                       T *__restrict__ y, int64_t rows,
                                                       int ncv) {
  typedef typename Vec16<T>::type V;
  constexpr int W = Vec16<T>::n, R = kGeluRows;
  const int cv = blockIdx.x * kGeluBlock + threadIdx.x;
  if (cv >= ncv) return;
  const V *xv = reinterpret_cast<const V *>(x);
  V *yv = reinterpret_cast<V *>(y);
  V b;
  if (BIAS) b = reinterpret_cast<const V *>(bias)[cv];
  for (int64_t r0 = (int64_t)blockIdx.y * R; r0 < rows; r0 += (int64_t)gridDim.y * R) {
    V v[R];
#pragma unroll
    for (int u = 0; u < R; ++u)
      if (r0 + u < rows) v[u] = __builtin_nontemporal_load(xv + (r0 + u) * ncv + cv);
    // the bias is opaque until the rows are requested: converted before the
    // loop, it was waited for before the first row load was issued
    if (BIAS) asm volatile("" : "+v"(b));
#pragma unroll
    for (int u = 0; u < R; ++u) {
      if (r0 + u < rows) {
        V o;
#pragma unroll
        for (int j = 0; j < W; ++j) {
          float f = (float)v[u][j];
          if (BIAS) f += (float)b[j];
          o[j] = (T)gelu<T, MODE>(f);
        }
        store_nt(yv + (r0 + u) * ncv + cv, o);
      }
    }
  }
}

template <typename T, int MODE, bool BIAS>
__global__ void gelu_scalar(const T *__restrict__ x, const T *__restrict__ bias,
                            T *__restrict__ y, int64_t n, int64_t cols) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += stride) {
    float f = (float)x[i];
    if (BIAS) f += (float)bias[i % cols];
    y[i] = (T)gelu<T, MODE>(f);
  }
}

template <typename T, int MODE, bool BIAS>
static void gelu_launch(const T *x, const T *bias, T *y, int64_t n,
                        int64_t cols, hipStream_t s) {
  constexpr int W = Vec16<T>::n;
  const bool vec = aligned16(x) && aligned16(y) && cols % W == 0 && cols / W < (1 << 30) &&
                   (!BIAS || aligned16(bias));
  if (vec) {
    const int64_t rows = n / cols;
    const int ncv = (int)(cols / W);
    const int64_t gy = (rows + kGeluRows - 1) / kGeluRows;
    dim3 grid((unsigned)((ncv + kGeluBlock - 1) / kGeluBlock), (unsigned)(gy > 65535 ? 65535 : gy));
    gelu_rows<T, MODE, BIAS><<<grid, kGeluBlock, 0, s>>>(x, bias, y, rows, ncv);
  } else
    gelu_scalar<T, MODE, BIAS><<<grid_for(n, 256), 256, 0, s>>>(x, bias, y, n, cols);
}

template <typename T>
static int gelu_impl(const void *x, const void *bias, void *y, int64_t n,
                     int64_t cols, int mode, hipStream_t s) {
  const T *xp = (const T *)x, *bp = (const T *)bias;
  T *yp = (T *)y;
  if (mode == ZK_GELU_ERF) {
    if (bp) gelu_launch<T, ZK_GELU_ERF, true>(xp, bp, yp, n, cols, s);
    else gelu_launch<T, ZK_GELU_ERF, false>(xp, bp, yp, n, cols, s);
  } else {
    if (bp) gelu_launch<T, ZK_GELU_TANH, true>(xp, bp, yp, n, cols, s);
    else gelu_launch<T, ZK_GELU_TANH, false>(xp, bp, yp, n, cols, s);
  }
  return check_launch("zk_gelu");
}

// -------------------------------------------------------------- quantise --

__global__ void quant_f16_vec(const f16 *__restrict__ x, int8_t *__restrict__ q,
                              int64_t nvec, float scale) {
  const float inv = 1.0f / scale;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nvec;
       i += stride) {
    f16x8 v = reinterpret_cast<const f16x8 *>(x)[i];
    float vf[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) vf[j] = (float)v[j];
    store_nt(reinterpret_cast<u32x2 *>(q) + i, quant8(vf, scale, inv));
  }
}

template <typename T>
__global__ void quant_scalar(const T *__restrict__ x, int8_t *__restrict__ q,
                             int64_t begin, int64_t n, float scale) {
  const float inv = 1.0f / scale;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = begin + blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
       i < n; i += stride)
    q[i] = quant1((float)x[i], scale, inv);
}

// ------------------------------------------------------------- transpose --
// 64x64 tile through LDS; scalar, bounds-checked accesses that are coalesced
// along the fast axis on both sides.
__global__ void transpose_f16_kernel(const f16 *__restrict__ src,
                                     f16 *__restrict__ dst, int64_t rows,
                                     int64_t cols, int64_t lds, int64_t ldd) {
  __shared__ f16 tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
  for (int r = ty; r < 64; r += 4) {
    const int64_t gr = r0 + r, gc = c0 + tx;
    tile[r][tx] = (gr < rows && gc < cols) ? src[gr * lds + gc] : (f16)0;
  }
  __syncthreads();
  for (int c = ty; c < 64; c += 4) {
    const int64_t gc = c0 + c, gr = r0 + tx;  // dst row = source column
    if (gc < cols && gr < rows) dst[gc * ldd + gr] = tile[tx][c];
  }
}

}  // namespace zk

using namespace zk;

extern "C" int zk_relu(const void *x, void *y, int64_t n, int dtype,
                       void *stream) {
  return unary_entry<kRelu>(x, y, n, dtype, stream, "zk_relu");
}

extern "C" int zk_sigmoid(const void *x, void *y, int64_t n, int dtype,
                          void *stream) {
  return unary_entry<kSigmoid>(x, y, n, dtype, stream, "zk_sigmoid");
}

extern "C" int zk_tanh(const void *x, void *y, int64_t n, int dtype,
                       void *stream) {
  return unary_entry<kTanh>(x, y, n, dtype, stream, "zk_tanh");
}

extern "C" int zk_gelu(const void *x, const void *bias, void *y, int64_t rows,
                       int64_t cols, int mode, int dtype, void *stream) {
  if (rows < 0 || cols < 0) return fail(ZK_ERR_INVALID, "zk_gelu: negative size");
  if (rows == 0 || cols == 0) return ZK_OK;
  if (!x || !y) return fail(ZK_ERR_INVALID, "zk_gelu: null pointer");
  if (mode != ZK_GELU_TANH && mode != ZK_GELU_ERF)
    return fail(ZK_ERR_INVALID, "zk_gelu: bad mode %d", mode);
  const int64_t n = rows * cols;
  if (dtype == ZK_F32) return gelu_impl<float>(x, bias, y, n, cols, mode, as_stream(stream));
  if (dtype == ZK_F16) return gelu_impl<f16>(x, bias, y, n, cols, mode, as_stream(stream));
  return fail(ZK_ERR_UNSUPPORTED, "zk_gelu: dtype %d not supported", dtype);
}

extern "C" int zk_quantize_i8(const void *x, int8_t *q, int64_t n, float scale,
                              int dtype, void *stream) {
  if (n < 0) return fail(ZK_ERR_INVALID, "zk_quantize_i8: negative size");
  if (n == 0) return ZK_OK;
  if (!x || !q) return fail(ZK_ERR_INVALID, "zk_quantize_i8: null pointer");
  if (!(scale > 0.0f) || scale != scale || scale == __builtin_inff())
    return fail(ZK_ERR_INVALID, "zk_quantize_i8: scale must be finite and > 0");
  hipStream_t s = as_stream(stream);
  if (dtype == ZK_F16) {
    const int64_t nvec =
        (aligned16(x) && (reinterpret_cast<uintptr_t>(q) & 7u) == 0) ? n / 8 : 0;
    if (nvec > 0)
      quant_f16_vec<<<grid_for(nvec, 256), 256, 0, s>>>((const f16 *)x, q, nvec, scale);
    if (nvec * 8 < n)
      quant_scalar<f16><<<grid_for(n - nvec * 8, 256), 256, 0, s>>>(
          (const f16 *)x, q, nvec * 8, n, scale);
  } else if (dtype == ZK_F32) {
    quant_scalar<float><<<grid_for(n, 256), 256, 0, s>>>((const float *)x, q, 0, n, scale);
  } else {
    return fail(ZK_ERR_UNSUPPORTED, "zk_quantize_i8: dtype %d not supported", dtype);
  }
  return check_launch("zk_quantize_i8");
}

extern "C" int zk_transpose_f16(const void *src, void *dst, int64_t rows,
                                int64_t cols, int64_t lds, int64_t ldd,
                                void *stream) {
  if (rows < 0 || cols < 0) return fail(ZK_ERR_INVALID, "zk_transpose_f16: negative size");
  if (rows == 0 || cols == 0) return ZK_OK;
  if (!src || !dst) return fail(ZK_ERR_INVALID, "zk_transpose_f16: null pointer");
  if (lds < cols || ldd < rows)
    return fail(ZK_ERR_INVALID, "zk_transpose_f16: leading dimension too small");
  if ((cols + 63) / 64 > 0x7fffffff || (rows + 63) / 64 > 65535)
    return fail(ZK_ERR_UNSUPPORTED, "zk_transpose_f16: matrix too large");
  dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
  transpose_f16_kernel<<<grid, 256, 0, as_stream(stream)>>>(
      (const f16 *)src, (f16 *)dst, rows, cols, lds, ldd);
  return check_launch("zk_transpose_f16");
}

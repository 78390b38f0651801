// Layout and small elementwise kernels for the GPU-resident tensor API:
// row-broadcast add, row softmax, the [d0,d1,d2,d3] -> [d0,d2,d1,d3]
// transpose of attention heads, and fp32 <-> fp16 conversion.
//
// All are bandwidth-bound. Accesses are 16-byte vectors where the layout
// allows (row length a multiple of the vector width, aligned pointers),
// scalar otherwise; fp16 arithmetic is done in fp32 and rounded once.
#include <type_traits>

#include "zk_common.hpp"

namespace zk {

namespace {

template <typename T> struct V16;
template <> struct V16<f16> { typedef f16x8 type; static constexpr int n = 8; };
template <> struct V16<float> { typedef f32x4 type; static constexpr int n = 4; };

inline unsigned blocks_for(int64_t work, int block) {
  int64_t g = (work + block - 1) / block;
  if (g > 65536) g = 65536;  // grid-stride loops cover the rest
  return (unsigned)(g < 1 ? 1 : g);
}

// ------------------------------------------------------------------ add --
// c[r, :] = a[r, :] + b[BCAST ? 0 : r, :]
template <typename T, bool BCAST>
__global__ void add_vec(const T *__restrict__ a, const T *__restrict__ b, T *__restrict__ c,
                        int64_t nvec, int64_t cvec) {
  typedef typename V16<T>::type V;
  constexpr int W = V16<T>::n;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nvec; i += stride) {
    const V x = reinterpret_cast<const V *>(a)[i];
    const V y = reinterpret_cast<const V *>(b)[BCAST ? i % cvec : i];
    V o;
#pragma unroll
    for (int j = 0; j < W; ++j) o[j] = (T)((float)x[j] + (float)y[j]);
    reinterpret_cast<V *>(c)[i] = o;
  }
}

template <typename T, bool BCAST>
__global__ void add_scalar(const T *__restrict__ a, const T *__restrict__ b, T *__restrict__ c,
                           int64_t n, int64_t cols) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += stride)
    c[i] = (T)((float)a[i] + (float)b[BCAST ? i % cols : i]);
}

template <typename T>
int add_impl(const void *a, const void *b, void *c, int64_t rows, int64_t cols, bool bcast,
             hipStream_t s) {
  constexpr int W = V16<T>::n;
  const int64_t n = rows * cols;
  const bool vec = cols % W == 0 && aligned16(a) && aligned16(b) && aligned16(c);
  const T *ap = (const T *)a, *bp = (const T *)b;
  T *cp = (T *)c;
  if (vec) {
    const unsigned g = blocks_for(n / W, 256);
    if (bcast) add_vec<T, true><<<g, 256, 0, s>>>(ap, bp, cp, n / W, cols / W);
    else add_vec<T, false><<<g, 256, 0, s>>>(ap, bp, cp, n / W, cols / W);
  } else {
    const unsigned g = blocks_for(n, 256);
    if (bcast) add_scalar<T, true><<<g, 256, 0, s>>>(ap, bp, cp, n, cols);
    else add_scalar<T, false><<<g, 256, 0, s>>>(ap, bp, cp, n, cols);
  }
  return check_launch("zk_add");
}

// -------------------------------------------------------------- softmax --
// One wavefront per row, three passes (max, sum of exp, normalise); the row
// is re-read from cache. expf and the division are the exact fp32 forms.
constexpr int kSmWaves = 4;

template <typename T>
__global__ __launch_bounds__(kSmWaves * kWave) void softmax_rows_kernel(
    const T *__restrict__ x, T *__restrict__ y, int64_t rows, int64_t cols) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * kSmWaves + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wavefront leaves together
  const T *xr = x + row * cols;
  T *yr = y + row * cols;
  float m = -__builtin_inff();
  for (int64_t j = lane; j < cols; j += kWave) m = fmaxf(m, (float)xr[j]);
  m = wave_max(m);
  float sum = 0.f;
  for (int64_t j = lane; j < cols; j += kWave) sum += expf((float)xr[j] - m);
  sum = wave_sum(sum);
  // (a row of -inf gives NaN, as the reference's and torch's softmax do)
  for (int64_t j = lane; j < cols; j += kWave) yr[j] = (T)(expf((float)xr[j] - m) / sum);
}

// ------------------------------------------------------ 0213 transpose --
// y[i][k][j][l] = x[i][j][k][l] for x of shape [d0, d1, d2, d3]; one thread
// per 16-byte vector of the contiguous last dimension.
template <typename T, bool VEC>
__global__ void transpose0213_kernel(const T *__restrict__ x, T *__restrict__ y, int64_t d0,
                                     int64_t d1, int64_t d2, int64_t d3u, int64_t total) {
  typedef typename V16<T>::type V;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total; t += stride) {
    // t indexes the OUTPUT [i][k][j][l] in units of d3u (vectors or scalars)
    const int64_t l = t % d3u;
    int64_t r = t / d3u;
    const int64_t j = r % d1;
    r /= d1;
    const int64_t k = r % d2;
    const int64_t i = r / d2;
    const int64_t src = ((i * d1 + j) * d2 + k) * d3u + l;
    if (VEC) reinterpret_cast<V *>(y)[t] = reinterpret_cast<const V *>(x)[src];
    else y[t] = x[src];
  }
  (void)d0;
}

template <typename T>
int transpose_impl(const void *x, void *y, int64_t d0, int64_t d1, int64_t d2, int64_t d3,
                   hipStream_t s) {
  constexpr int W = V16<T>::n;
  const bool vec = d3 % W == 0 && aligned16(x) && aligned16(y);
  if (vec) {
    const int64_t total = d0 * d1 * d2 * (d3 / W);
    transpose0213_kernel<T, true><<<blocks_for(total, 256), 256, 0, s>>>(
        (const T *)x, (T *)y, d0, d1, d2, d3 / W, total);
  } else {
    const int64_t total = d0 * d1 * d2 * d3;
    transpose0213_kernel<T, false><<<blocks_for(total, 256), 256, 0, s>>>(
        (const T *)x, (T *)y, d0, d1, d2, d3, total);
  }
  return check_launch("zk_transpose_0213");
}

// -------------------------------------------------------------- convert --
template <typename S, typename D>
__global__ void convert_kernel(const S *__restrict__ x, D *__restrict__ y, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  // four elements per thread per pass (8 or 16 bytes in, 8 or 16 out)
  for (int64_t i = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) * 4; i < n; i += stride * 4) {
    if (i + 4 <= n) {
#pragma unroll
      for (int j = 0; j < 4; ++j) y[i + j] = (D)(float)x[i + j];
    } else {
      for (int64_t j = i; j < n; ++j) y[j] = (D)(float)x[j];
    }
  }
}

}  // namespace
}  // namespace zk

using namespace zk;

extern "C" int zk_add(const void *a, const void *b, void *c, int64_t rows, int64_t cols,
                      int64_t b_rows, int dtype, void *stream) {
  if (rows < 0 || cols < 0) return fail(ZK_ERR_INVALID, "zk_add: negative size");
  if (rows == 0 || cols == 0) return ZK_OK;
  if (!a || !b || !c) return fail(ZK_ERR_INVALID, "zk_add: null pointer");
  if (b_rows != 1 && b_rows != rows)
    return fail(ZK_ERR_INVALID, "zk_add: b must have 1 or %lld rows", (long long)rows);
  const bool bcast = b_rows == 1 && rows > 1;
  hipStream_t s = as_stream(stream);
  if (dtype == ZK_F32) return add_impl<float>(a, b, c, rows, cols, bcast, s);
  if (dtype == ZK_F16) return add_impl<f16>(a, b, c, rows, cols, bcast, s);
  return fail(ZK_ERR_UNSUPPORTED, "zk_add: dtype %d not supported", dtype);
}

extern "C" int zk_softmax(const void *x, void *y, int64_t rows, int64_t cols, int dtype,
                          void *stream) {
  if (rows < 0 || cols < 0) return fail(ZK_ERR_INVALID, "zk_softmax: negative size");
  if (rows == 0 || cols == 0) return ZK_OK;
  if (!x || !y) return fail(ZK_ERR_INVALID, "zk_softmax: null pointer");
  if ((rows + kSmWaves - 1) / kSmWaves > 0x7fffffff)
    return fail(ZK_ERR_UNSUPPORTED, "zk_softmax: too many rows");
  const unsigned g = (unsigned)((rows + kSmWaves - 1) / kSmWaves);
  hipStream_t s = as_stream(stream);
  if (dtype == ZK_F32)
    softmax_rows_kernel<float><<<g, kSmWaves * kWave, 0, s>>>((const float *)x, (float *)y, rows, cols);
  else if (dtype == ZK_F16)
    softmax_rows_kernel<f16><<<g, kSmWaves * kWave, 0, s>>>((const f16 *)x, (f16 *)y, rows, cols);
  else
    return fail(ZK_ERR_UNSUPPORTED, "zk_softmax: dtype %d not supported", dtype);
  return check_launch("zk_softmax");
}

extern "C" int zk_transpose_0213(const void *x, void *y, int64_t d0, int64_t d1, int64_t d2,
                                 int64_t d3, int dtype, void *stream) {
  if (d0 < 0 || d1 < 0 || d2 < 0 || d3 < 0)
    return fail(ZK_ERR_INVALID, "zk_transpose_0213: negative size");
  if (d0 == 0 || d1 == 0 || d2 == 0 || d3 == 0) return ZK_OK;
  if (!x || !y) return fail(ZK_ERR_INVALID, "zk_transpose_0213: null pointer");
  if (x == y) return fail(ZK_ERR_INVALID, "zk_transpose_0213: in-place is not supported");
  hipStream_t s = as_stream(stream);
  if (dtype == ZK_F32) return transpose_impl<float>(x, y, d0, d1, d2, d3, s);
  if (dtype == ZK_F16) return transpose_impl<f16>(x, y, d0, d1, d2, d3, s);
  return fail(ZK_ERR_UNSUPPORTED, "zk_transpose_0213: dtype %d not supported", dtype);
}

extern "C" int zk_convert(const void *x, void *y, int64_t n, int src_dtype, int dst_dtype,
                          void *stream) {
  if (n < 0) return fail(ZK_ERR_INVALID, "zk_convert: negative size");
  if (n == 0) return ZK_OK;
  if (!x || !y) return fail(ZK_ERR_INVALID, "zk_convert: null pointer");
  hipStream_t s = as_stream(stream);
  const unsigned g = blocks_for((n + 3) / 4, 256);
  if (src_dtype == ZK_F32 && dst_dtype == ZK_F16)
    convert_kernel<float, f16><<<g, 256, 0, s>>>((const float *)x, (f16 *)y, n);
  else if (src_dtype == ZK_F16 && dst_dtype == ZK_F32)
    convert_kernel<f16, float><<<g, 256, 0, s>>>((const f16 *)x, (float *)y, n);
  else
    return fail(ZK_ERR_UNSUPPORTED, "zk_convert: %d -> %d not supported", src_dtype, dst_dtype);
  return check_launch("zk_convert");
}

// LayerNorm and fused Add+LayerNorm (post-LN BERT residual), fp32 statistics.
//
// Fast path: one or two rows per wavefront. Each lane keeps its slice of the
// row in registers as 16-byte vectors, so the row is read from HBM exactly once
// (twice with the residual) and written once; mean and variance are exact
// two-pass statistics over the register copy, reduced with cross-lane
// butterflies. Rows whose hidden size is not a multiple of the vector width
// (or larger than the register budget) take a block-per-row kernel that
// re-reads the row from cache.
#include "zk_common.hpp"

namespace zk {

template <typename T> struct LnVec;
template <> struct LnVec<f16> { typedef f16x8 type; static constexpr int n = 8; };
template <> struct LnVec<float> { typedef f32x4 type; static constexpr int n = 4; };

constexpr int kLnWaves = 4;  // wavefronts per 256-thread block

// LPR lanes per row (64 / LPR rows per wavefront): a 768-wide fp16 row is 96
// 16-byte vectors, so two rows per wavefront give every lane exactly three.
template <typename T, int MAXV, bool RES, int LPR>
__global__ __launch_bounds__(kLnWaves * kWave) void ln_wave_kernel(
    const T *__restrict__ x, const T *__restrict__ res,
    const T *__restrict__ gamma, const T *__restrict__ beta, T *__restrict__ y,
    int64_t rows, int hidden, float eps) {
  typedef typename LnVec<T>::type V;
  constexpr int W = LnVec<T>::n;
  constexpr int RPW = kWave / LPR;  // rows per wavefront
  const int lane = threadIdx.x & (kWave - 1);
  const int sub = lane % LPR;
  const int64_t row = ((int64_t)blockIdx.x * kLnWaves + (threadIdx.x >> 6)) * RPW + lane / LPR;
  // Rows past the end load nothing and store nothing, but stay in the
  // shuffles (their partner lanes belong to the same row group).
  const bool live = row < rows;
  const int nvec = hidden / W;
  const V *xr = reinterpret_cast<const V *>(x + (live ? row : 0) * hidden);
  const V *rr = reinterpret_cast<const V *>(res + (RES && live ? row * hidden : 0));

  float v[MAXV][W];
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < MAXV; ++k) {
    const int idx = sub + k * LPR;
    if (live && idx < nvec) {
      V a = xr[idx];
      V r;
      if (RES) r = rr[idx];
#pragma unroll
      for (int j = 0; j < W; ++j) {
        float f = (float)a[j];
        if (RES) f += (float)r[j];
        v[k][j] = f;
        sum += f;
      }
    } else {
#pragma unroll
      for (int j = 0; j < W; ++j) v[k][j] = 0.f;
    }
  }
  auto group_sum = [](float t) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) t += __shfl_xor(t, o, kWave);
    return t;
  };
  const float inv_h = 1.0f / (float)hidden;
  const float mean = group_sum(sum) * inv_h;
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < MAXV; ++k) {
    if (sub + k * LPR < nvec) {
#pragma unroll
      for (int j = 0; j < W; ++j) {
        const float d = v[k][j] - mean;
        sq += d * d;
      }
    }
  }
  const float var = group_sum(sq) * inv_h;
  const float rstd = 1.0f / sqrtf(var + eps);
  if (!live) return;

  V *yr = reinterpret_cast<V *>(y + row * hidden);
  const V *gv = reinterpret_cast<const V *>(gamma);
  const V *bv = reinterpret_cast<const V *>(beta);
#pragma unroll
  for (int k = 0; k < MAXV; ++k) {
    const int idx = sub + k * LPR;
    if (idx < nvec) {
      V g = gv[idx], b = bv[idx], o;
#pragma unroll
      for (int j = 0; j < W; ++j)
        o[j] = (T)((v[k][j] - mean) * rstd * (float)g[j] + (float)b[j]);
      yr[idx] = o;
    }
  }
}

// Generic fallback: one 256-thread block per row, three passes over the row.
template <typename T, bool RES>
__global__ __launch_bounds__(256) void ln_block_kernel(
    const T *__restrict__ x, const T *__restrict__ res,
    const T *__restrict__ gamma, const T *__restrict__ beta, T *__restrict__ y,
    int64_t hidden, float eps) {
  __shared__ float part[256 / kWave];
  const int64_t row = blockIdx.x;
  const T *xr = x + row * hidden;
  const T *rr = RES ? res + row * hidden : nullptr;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid >> 6;
  constexpr int NW = 256 / kWave;

  auto block_sum = [&](float s) -> float {
    s = wave_sum(s);
    __syncthreads();  // previous readers of part[] are done
    if (lane == 0) part[wid] = s;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) t += part[i];
    return t;  // every thread holds the block total
  };

  float s = 0.f;
  for (int64_t i = tid; i < hidden; i += 256)
    s += (float)xr[i] + (RES ? (float)rr[i] : 0.f);
  const float mean = block_sum(s) / (float)hidden;
  float q = 0.f;
  for (int64_t i = tid; i < hidden; i += 256) {
    const float d = (float)xr[i] + (RES ? (float)rr[i] : 0.f) - mean;
    q += d * d;
  }
  const float rstd = 1.0f / sqrtf(block_sum(q) / (float)hidden + eps);
  for (int64_t i = tid; i < hidden; i += 256) {
    const float f = (float)xr[i] + (RES ? (float)rr[i] : 0.f);
    y[row * hidden + i] = (T)((f - mean) * rstd * (float)gamma[i] + (float)beta[i]);
  }
}

template <typename T, int MAXV, int LPR>
static void ln_wave_launch(const T *x, const T *r, const T *g, const T *b, T *y,
                           int64_t rows, int hidden, float eps, hipStream_t s) {
  constexpr int rows_per_block = kLnWaves * (kWave / LPR);
  const unsigned grid = (unsigned)((rows + rows_per_block - 1) / rows_per_block);
  if (r)
    ln_wave_kernel<T, MAXV, true, LPR><<<grid, kLnWaves * kWave, 0, s>>>(x, r, g, b, y, rows, hidden, eps);
  else
    ln_wave_kernel<T, MAXV, false, LPR><<<grid, kLnWaves * kWave, 0, s>>>(x, r, g, b, y, rows, hidden, eps);
}

template <typename T>
static int ln_impl(const void *xv, const void *rv, const void *gv,
                   const void *bv, void *yv, int64_t rows, int64_t hidden,
                   float eps, hipStream_t s) {
  const T *x = (const T *)xv, *r = (const T *)rv, *g = (const T *)gv,
          *b = (const T *)bv;
  T *y = (T *)yv;
  constexpr int W = LnVec<T>::n;
  const bool vec_ok = hidden % W == 0 && aligned16(x) && aligned16(y) &&
                      aligned16(g) && aligned16(b) && (!r || aligned16(r));
  const int64_t nvec = hidden / W;
  if (vec_ok && nvec <= 16 * kWave && (rows + kLnWaves - 1) / kLnWaves <= 0x7fffffff) {
    const int h = (int)hidden;
    // 32 lanes per row while a row fits in 4 vectors per lane (H <= 1024 in
    // fp16), else a whole wavefront per row.
    if (nvec <= 32) ln_wave_launch<T, 1, 32>(x, r, g, b, y, rows, h, eps, s);
    else if (nvec <= 64) ln_wave_launch<T, 2, 32>(x, r, g, b, y, rows, h, eps, s);
    else if (nvec <= 96) ln_wave_launch<T, 3, 32>(x, r, g, b, y, rows, h, eps, s);
    else if (nvec <= 128) ln_wave_launch<T, 4, 32>(x, r, g, b, y, rows, h, eps, s);
    else if (nvec <= 256) ln_wave_launch<T, 4, 64>(x, r, g, b, y, rows, h, eps, s);
    else if (nvec <= 512) ln_wave_launch<T, 8, 64>(x, r, g, b, y, rows, h, eps, s);
    else ln_wave_launch<T, 16, 64>(x, r, g, b, y, rows, h, eps, s);
  } else {
    if (rows > 0x7fffffff)
      return fail(ZK_ERR_UNSUPPORTED, "zk_layernorm: too many rows for the generic path");
    if (r)
      ln_block_kernel<T, true><<<(unsigned)rows, 256, 0, s>>>(x, r, g, b, y, hidden, eps);
    else
      ln_block_kernel<T, false><<<(unsigned)rows, 256, 0, s>>>(x, r, g, b, y, hidden, eps);
  }
  return check_launch("zk_layernorm");
}

}  // namespace zk

using namespace zk;

extern "C" int zk_layernorm(const void *x, const void *residual,
                            const void *gamma, const void *beta, void *y,
                            int64_t rows, int64_t hidden, float eps, int dtype,
                            void *stream) {
  if (rows < 0 || hidden < 0)
    return fail(ZK_ERR_INVALID, "zk_layernorm: negative size");
  if (rows == 0) return ZK_OK;
  if (hidden == 0) return fail(ZK_ERR_INVALID, "zk_layernorm: hidden must be > 0");
  if (!x || !gamma || !beta || !y)
    return fail(ZK_ERR_INVALID, "zk_layernorm: null pointer");
  if (!(eps >= 0.0f)) return fail(ZK_ERR_INVALID, "zk_layernorm: eps must be >= 0");
  hipStream_t s = as_stream(stream);
  if (dtype == ZK_F32) return ln_impl<float>(x, residual, gamma, beta, y, rows, hidden, eps, s);
  if (dtype == ZK_F16) return ln_impl<f16>(x, residual, gamma, beta, y, rows, hidden, eps, s);
  return fail(ZK_ERR_UNSUPPORTED, "zk_layernorm: dtype %d not supported", dtype);
}

// LayerNorm, fused Add+LayerNorm (post-LN BERT residual: LN(x + r)) and
// LayerNorm+Add (LN(x) + r, the reference's LayerNormAdd), fp32 statistics.
//
// Fast path: one or two rows per wavefront. Each lane keeps its slice of the
// row in registers as 16-byte vectors, so the row is read from HBM exactly once
// (twice with the residual) and written once; mean and variance are exact
// two-pass statistics over the register copy, reduced with cross-lane
// butterflies. Rows whose hidden size is not a multiple of the vector width
// (or larger than the register budget) take a block-per-row kernel that
// re-reads the row from cache.
#include <type_traits>

#include "zk_common.hpp"

namespace zk {

template <typename T> struct LnVec;
template <> struct LnVec<f16> { typedef f16x8 type; static constexpr int n = 8; };
template <> struct LnVec<float> { typedef f32x4 type; static constexpr int n = 4; };

constexpr int kLnWaves = 4;  // wavefronts per 256-thread block
// launches of at most this many wavefronts (16 per CU) read their rows with
// the loads batched (ln_wave_kernel's BATCH)
constexpr int kLnBatchWaves = 4096;

// Residual placement: none, added before the statistics (Add+LayerNorm),
// added to the normalised output (LayerNorm+Add), or added before the
// statistics as the LayerNorm of the given rows (kResPreLn: r' = (r - mean)
// rstd g + b with the per-row (mean, rstd) and g, b of that earlier
// LayerNorm, computed on the fly in fp32).
enum { kResNone = 0, kResPre = 1, kResPost = 2, kResPreLn = 3 };

// The earlier LayerNorm of the residual rows (kResPreLn).
template <typename T> struct ResLn {
  const float2 *ms;  // [rows] (mean, rstd)
  const T *g, *b;    // [hidden]
};

// PART (1 or 2): the input rows are not read from x but formed from the fp32
// split-K partials of a GEMM, [splits][rows][hidden] (split s at ws + s *
// stride), summed in split order from zero, plus the bias, rounded to T:
// exactly the values splitk_reduce (epilogue ZK_EPI_BIAS) would store for x.
// PART 1: each lane forms its own vectors. PART 2 (rows of at most 1024
// values, LPR = 64): one row per workgroup, whose four wavefronts form the
// row in LDS, after which wavefront 0 alone runs the LayerNorm on it, with
// the same arithmetic as for a row read from memory; for many splits of few
// rows, where one wavefront reading every split of its row is too slow.
template <typename T> struct PartIn {
  const float *ws;
  int splits;
  int64_t stride;
  const T *bias;  // [hidden]
};

// LPR lanes per row (64 / LPR rows per wavefront): a 768-wide fp16 row is 96
// 16-byte vectors, so two rows per wavefront give every lane exactly three.
// Q8: also write q = quant(y) as int8 (the fp16 output value quantised with
// scale qs), for an int8 GEMM that consumes the normalised rows.
template <typename T, int MAXV, int RES, int LPR, bool Q8, int PART = 0, bool BATCH = false>
__global__ __launch_bounds__(kLnWaves * kWave) void ln_wave_kernel(
    const T *__restrict__ x, const T *__restrict__ res,
    const T *__restrict__ gamma, const T *__restrict__ beta, T *__restrict__ y,
    int8_t *__restrict__ q, float qs, int64_t rows, int hidden, float eps, ResLn<T> rl,
    PartIn<T> pin) {
  constexpr bool PRE = RES == kResPre || RES == kResPreLn;
  typedef typename LnVec<T>::type V;
  constexpr int W = LnVec<T>::n;
  constexpr int RPW = kWave / LPR;  // rows per wavefront
  const int lane = threadIdx.x & (kWave - 1);
  const int sub = lane % LPR;
  const int64_t row = PART == 2
                          ? (int64_t)blockIdx.x
                          : ((int64_t)blockIdx.x * kLnWaves + (threadIdx.x >> 6)) * RPW + lane / LPR;
  // Rows past the end load nothing and store nothing, but stay in the
  // shuffles (their partner lanes belong to the same row group).
  const bool live = row < rows;
  const int nvec = hidden / W;
  __shared__ V prow[PART == 2 ? 128 : 1];
  if constexpr (PART == 2) {
    static_assert(W == 8 && LPR == kWave && MAXV <= 2, "one wavefront per row of <= 128 vectors");
    // the row's values from the partials, four columns per thread
    const float *pp = pin.ws + row * hidden;
    for (int c = threadIdx.x; c < hidden / 4; c += kLnWaves * kWave) {
      const f16x4 bias = *(const f16x4 *)(pin.bias + 4 * c);
      const f32x4 t = sum_splits<f32x4>(pp + 4 * c, pin.splits, pin.stride);
      f16x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = (T)as_f32(t[j] + (float)bias[j]);
      *(f16x4 *)(reinterpret_cast<f16 *>(prow) + 4 * c) = o;
    }
    __syncthreads();
    if (threadIdx.x >= kWave) return;
  }
  const V *xr = reinterpret_cast<const V *>(x + (live ? row : 0) * hidden);
  const V *rr = reinterpret_cast<const V *>(res + (RES != kResNone && live ? row * hidden : 0));
  float2 rms = make_float2(0.f, 1.f);
  if constexpr (RES == kResPreLn) rms = rl.ms[live ? row : 0];

  const V *gv = reinterpret_cast<const V *>(gamma);
  const V *bv = reinterpret_cast<const V *>(beta);
  // BATCHED (rows read from memory by launches of at most kLnBatchWaves
  // wavefronts, or formed in LDS): loads are issued ahead of their use, each
  // from a valid
  // address (row 0, vector 0 where the lane has nothing to read): the row's
  // vectors (and residual) four at a time, and, for rows of at most four
  // vectors per lane, the output's gamma / beta (and post residual) at the
  // start, so that a wavefront waits for memory about once rather than once
  // per load. In a launch of one round of wavefronts that wait is the
  // kernel's critical path ([4096, 768] Add+LN 6.5 -> 5.4 us); with several
  // rounds the other wavefronts hide it, and one load at a time per
  // wavefront was faster ([16384, 768] 13.9 us against 14.8 us batched).
  constexpr int CH = MAXV < 4 ? MAXV : 4;
  constexpr bool BATCHED = (PART == 0 && BATCH) || PART == 2;  // PART 2: row in LDS
  constexpr bool PRE_OUT = BATCHED && MAXV <= 4;
  V go[PRE_OUT ? MAXV : 1], bo[PRE_OUT ? MAXV : 1], ro[PRE_OUT && RES == kResPost ? MAXV : 1];
  if constexpr (PRE_OUT) {
#pragma unroll
    for (int k = 0; k < MAXV; ++k) {
      const int idx = sub + k * LPR, ci = idx < nvec ? idx : 0;
      go[k] = gv[ci];
      bo[k] = bv[ci];
      if constexpr (RES == kResPost) ro[k] = rr[ci];
    }
  }
  float v[MAXV][W];
  float sum = 0.f;
  // the input value of one vector: a (+ r, or + LN(r) with gamma rg, beta rb)
  auto combine = [&](const V &a, const V &r, const V &rg, const V &rb, float (&f)[W]) {
#pragma unroll
    for (int j = 0; j < W; ++j) {
      f[j] = (float)a[j];
      if constexpr (RES == kResPre) f[j] += (float)r[j];
      if constexpr (RES == kResPreLn)
        f[j] += fmaf(((float)r[j] - rms.x) * rms.y, (float)rg[j], (float)rb[j]);
    }
  };
  if constexpr (BATCHED) {
    // Branch-free: a lane with no vector k combines what it loaded from vector
    // 0 and keeps zeros (adding 0 leaves the sum as it is).
#pragma unroll
    for (int k0 = 0; k0 < MAXV; k0 += CH) {
      V xa[CH], xq[CH], xg[CH], xb[CH];
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int idx = sub + (k0 + c) * LPR, ci = live && idx < nvec ? idx : 0;
        if constexpr (PART == 2) xa[c] = prow[ci];
        else xa[c] = xr[ci];
        if constexpr (PRE) xq[c] = rr[ci];
        if constexpr (RES == kResPreLn) {
          xg[c] = reinterpret_cast<const V *>(rl.g)[ci];
          xb[c] = reinterpret_cast<const V *>(rl.b)[ci];
        }
      }
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int k = k0 + c;
        const bool ok = live && sub + k * LPR < nvec;
        float f[W];
        combine(xa[c], xq[c], xg[c], xb[c], f);
#pragma unroll
        for (int j = 0; j < W; ++j) {
          v[k][j] = ok ? f[j] : 0.f;
          sum += v[k][j];
        }
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < MAXV; ++k) {
      const int idx = sub + k * LPR;
      if (live && idx < nvec) {
        V a;
        if constexpr (PART == 0) {
          a = xr[idx];
        } else {
          static_assert(W == 8, "partials are summed 8 columns at a time");
          const float *pp = pin.ws + (row * hidden + (int64_t)idx * W);
          const f32x4 lo = sum_splits<f32x4>(pp, pin.splits, pin.stride);
          const f32x4 hi = sum_splits<f32x4>(pp + 4, pin.splits, pin.stride);
          const V bias = reinterpret_cast<const V *>(pin.bias)[idx];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            a[j] = (T)as_f32(lo[j] + (float)bias[j]);
            a[j + 4] = (T)as_f32(hi[j] + (float)bias[j + 4]);
          }
        }
        V r, rg, rb;
        if constexpr (PRE) r = rr[idx];
        if constexpr (RES == kResPreLn) {
          rg = reinterpret_cast<const V *>(rl.g)[idx];
          rb = reinterpret_cast<const V *>(rl.b)[idx];
        }
        float f[W];
        combine(a, r, rg, rb, f);
#pragma unroll
        for (int j = 0; j < W; ++j) {
          v[k][j] = f[j];
          sum += f[j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < W; ++j) v[k][j] = 0.f;
      }
    }
  }
  auto group_sum = [](float t) { return group_reduce<LPR>(t, OpAdd{}); };
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
#pragma unroll
  for (int k = 0; k < MAXV; ++k) {
    const int idx = sub + k * LPR;
    if (idx < nvec) {
      V g, b, o;
      if constexpr (PRE_OUT) {
        g = go[k];
        b = bo[k];
      } else {
        g = gv[idx];
        b = bv[idx];
      }
      if constexpr (RES == kResPost) {
        V r;
        if constexpr (PRE_OUT) r = ro[k];
        else r = rr[idx];
#pragma unroll
        for (int j = 0; j < W; ++j)
          o[j] = (T)as_f32((v[k][j] - mean) * rstd * (float)g[j] + (float)b[j] + (float)r[j]);
      } else {
#pragma unroll
        for (int j = 0; j < W; ++j)
          o[j] = (T)as_f32((v[k][j] - mean) * rstd * (float)g[j] + (float)b[j]);
      }
      store_nt(yr + idx, o);
      if constexpr (Q8) {
        static_assert(W == 8, "int8 output is written 8 bytes per vector");
        float of[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) of[j] = (float)o[j];
        store_nt(reinterpret_cast<u32x2 *>(q + row * hidden) + idx, quant8(of, qs, 1.0f / qs));
      }
    }
  }
}

// Generic fallback: one 256-thread block per row, three passes over the row.
template <typename T, int RES, bool Q8>
__global__ __launch_bounds__(256) void ln_block_kernel(
    const T *__restrict__ x, const T *__restrict__ res,
    const T *__restrict__ gamma, const T *__restrict__ beta, T *__restrict__ y,
    int8_t *__restrict__ q, float qs, int64_t hidden, float eps, ResLn<T> rl) {
  __shared__ float part[256 / kWave];
  const int64_t row = blockIdx.x;
  const T *xr = x + row * hidden;
  const T *rr = RES != kResNone ? res + row * hidden : nullptr;
  constexpr bool PRE = RES == kResPre || RES == kResPreLn;
  const float2 rms = RES == kResPreLn ? rl.ms[row] : make_float2(0.f, 1.f);
  // the residual's value at column i (kResPreLn: its LayerNorm)
  auto rv = [&](int64_t i) {
    if constexpr (RES == kResPreLn)
      return fmaf(((float)rr[i] - rms.x) * rms.y, (float)rl.g[i], (float)rl.b[i]);
    return (float)rr[i];
  };
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
    s += (float)xr[i] + (PRE ? rv(i) : 0.f);
  const float mean = block_sum(s) / (float)hidden;
  float sq = 0.f;
  for (int64_t i = tid; i < hidden; i += 256) {
    const float d = (float)xr[i] + (PRE ? rv(i) : 0.f) - mean;
    sq += d * d;
  }
  const float rstd = 1.0f / sqrtf(block_sum(sq) / (float)hidden + eps);
  for (int64_t i = tid; i < hidden; i += 256) {
    const float f = (float)xr[i] + (PRE ? rv(i) : 0.f);
    float yv = (f - mean) * rstd * (float)gamma[i] + (float)beta[i];
    if (RES == kResPost) yv += (float)rr[i];
    const T o = (T)as_f32(yv);
    y[row * hidden + i] = o;
    if (Q8) q[row * hidden + i] = quant1((float)o, qs, 1.0f / qs);
  }
}

template <typename T, int MAXV, int LPR, bool Q8>
static void ln_wave_launch(const T *x, const T *r, const T *g, const T *b, T *y, int8_t *q,
                           float qs, int64_t rows, int hidden, float eps, bool post,
                           ResLn<T> rl, hipStream_t s) {
  constexpr int rows_per_block = kLnWaves * (kWave / LPR);
  const unsigned grid = (unsigned)((rows + rows_per_block - 1) / rows_per_block);
  const bool batch = (int64_t)grid * kLnWaves <= kLnBatchWaves;
#define ZK_LNW(RES, QQ)                                                                        \
  do {                                                                                         \
    if (batch)                                                                                 \
      ln_wave_kernel<T, MAXV, RES, LPR, QQ, 0, true><<<grid, kLnWaves * kWave, 0, s>>>(        \
          x, r, g, b, y, q, qs, rows, hidden, eps, rl, PartIn<T>{});                           \
    else                                                                                       \
      ln_wave_kernel<T, MAXV, RES, LPR, QQ><<<grid, kLnWaves * kWave, 0, s>>>(                 \
          x, r, g, b, y, q, qs, rows, hidden, eps, rl, PartIn<T>{});                           \
  } while (0)
  if (r && post) {
    if constexpr (!Q8) ZK_LNW(kResPost, false);
  } else if (r && rl.ms) {
    if constexpr (Q8) ZK_LNW(kResPreLn, true);
  } else if (r) {
    ZK_LNW(kResPre, Q8);
  } else {
    ZK_LNW(kResNone, Q8);
  }
#undef ZK_LNW
}

// (vectors per lane MAXV, lanes per row LPR) of the wave kernel for `rows`
// rows of `nvec` vectors (nvec <= 16 * 64): every launch of a given shape,
// from rows or from split-K partials, takes its shape from here and so sums
// in one order. With few rows (under 2048: a few sequences) a whole
// wavefront per row gives four rows per workgroup instead of eight, twice
// the workgroups.
template <class F>
static void ln_pick(int64_t rows, int64_t nvec, F &&launch) {
  using std::integral_constant;
  const bool few = rows < 2048;
  if (few && nvec <= 64) launch(integral_constant<int, 1>(), integral_constant<int, 64>());
  else if (few && nvec <= 128) launch(integral_constant<int, 2>(), integral_constant<int, 64>());
  else if (nvec <= 32) launch(integral_constant<int, 1>(), integral_constant<int, 32>());
  else if (nvec <= 64) launch(integral_constant<int, 2>(), integral_constant<int, 32>());
  else if (nvec <= 96) launch(integral_constant<int, 3>(), integral_constant<int, 32>());
  else if (nvec <= 128) launch(integral_constant<int, 4>(), integral_constant<int, 32>());
  else if (nvec <= 256) launch(integral_constant<int, 4>(), integral_constant<int, 64>());
  else if (nvec <= 512) launch(integral_constant<int, 8>(), integral_constant<int, 64>());
  else launch(integral_constant<int, 16>(), integral_constant<int, 64>());
}

// post: the residual is added after normalisation (LN(x) + r) instead of
// before it (LN(x + r)); never combined with the int8 output. rl.ms set: the
// residual is the LayerNorm of r (int8 output only).
template <typename T, bool Q8>
static int ln_impl(const void *xv, const void *rv, const void *gv,
                   const void *bv, void *yv, int8_t *q, float qs, int64_t rows,
                   int64_t hidden, float eps, hipStream_t s, bool post = false,
                   ResLn<T> rl = ResLn<T>{nullptr, nullptr, nullptr}) {
  const T *x = (const T *)xv, *r = (const T *)rv, *g = (const T *)gv,
          *b = (const T *)bv;
  T *y = (T *)yv;
  constexpr int W = LnVec<T>::n;
  const bool vec_ok = hidden % W == 0 && aligned16(x) && aligned16(y) &&
                      aligned16(g) && aligned16(b) && (!r || aligned16(r)) &&
                      (!Q8 || aligned8(q)) && (!rl.ms || (aligned16(rl.g) && aligned16(rl.b)));
  const int64_t nvec = hidden / W;
  if (vec_ok && nvec <= 16 * kWave && (rows + kLnWaves - 1) / kLnWaves <= 0x7fffffff) {
    const int h = (int)hidden;
    // 32 lanes per row while a row fits in 4 vectors per lane (H <= 1024 in
    // fp16), else a whole wavefront per row.
    ln_pick(rows, nvec, [&](auto mv, auto lpr) {
      ln_wave_launch<T, decltype(mv)::value, decltype(lpr)::value, Q8>(x, r, g, b, y, q, qs, rows,
                                                                      h, eps, post, rl, s);
    });
  } else {
    if (rows > 0x7fffffff)
      return fail(ZK_ERR_UNSUPPORTED, "zk_layernorm: too many rows for the generic path");
#define ZK_LNB(RES, QQ) \
  ln_block_kernel<T, RES, QQ><<<(unsigned)rows, 256, 0, s>>>(x, r, g, b, y, q, qs, hidden, eps, rl)
    if (r && post) {
      if constexpr (!Q8) ZK_LNB(kResPost, false);
    } else if (r && rl.ms) {
      if constexpr (Q8) ZK_LNB(kResPreLn, true);
    } else if (r) {
      ZK_LNB(kResPre, Q8);
    } else {
      ZK_LNB(kResNone, Q8);
    }
#undef ZK_LNB
  }
  return check_launch("zk_layernorm");
}

bool ln_partials_ok(const float *ws, int64_t stride, const void *bias, const void *res,
                    const void *g, const void *b, const void *y, int64_t rows, int64_t hidden) {
  return hidden > 0 && hidden % 8 == 0 && hidden / 8 <= 16 * kWave && stride % 4 == 0 &&
         (rows + kLnWaves - 1) / kLnWaves <= 0x7fffffff && aligned16(ws) && aligned16(bias) &&
         aligned16(res) && aligned16(g) && aligned16(b) && aligned16(y);
}

bool ln_partials_wide_ok(int64_t rows, int64_t hidden) {
  return rows < 2048 && hidden <= 1024;  // ln_pick's one-wavefront-per-row shapes
}

int ln_add_partials_f16(const float *ws, int splits, int64_t stride, const void *bias,
                        const void *res, const void *g, const void *b, void *y, int64_t rows,
                        int64_t hidden, float eps, bool wide, hipStream_t s) {
  const PartIn<f16> pin{ws, splits, stride, (const f16 *)bias};
  const int h = (int)hidden;
  ln_pick(rows, hidden / 8, [&](auto mv, auto lpr) {
    constexpr int MV = decltype(mv)::value, LPR = decltype(lpr)::value;
    constexpr int rows_per_block = kLnWaves * (kWave / LPR);
    const ResLn<f16> none{nullptr, nullptr, nullptr};
    if constexpr (LPR == kWave && MV <= 2) {
      if (wide) {
        ln_wave_kernel<f16, MV, kResPre, LPR, false, 2><<<(unsigned)rows, kLnWaves * kWave, 0, s>>>(
            nullptr, (const f16 *)res, (const f16 *)g, (const f16 *)b, (f16 *)y, nullptr, 1.f,
            rows, h, eps, none, pin);
        return;
      }
    }
    const unsigned grid = (unsigned)((rows + rows_per_block - 1) / rows_per_block);
    ln_wave_kernel<f16, MV, kResPre, LPR, false, 1><<<grid, kLnWaves * kWave, 0, s>>>(
        nullptr, (const f16 *)res, (const f16 *)g, (const f16 *)b, (f16 *)y, nullptr, 1.f, rows,
        h, eps, none, pin);
  });
  return check_launch("zk_gemm_f16_add_ln");
}

}  // namespace zk

using namespace zk;

static int ln_check(const char *who, const void *x, const void *gamma, const void *beta,
                    const void *y, int64_t rows, int64_t hidden, float eps) {
  if (rows < 0 || hidden < 0) return fail(ZK_ERR_INVALID, "%s: negative size", who);
  if (rows == 0) return ZK_OK;
  if (hidden == 0) return fail(ZK_ERR_INVALID, "%s: hidden must be > 0", who);
  if (!x || !gamma || !beta || !y) return fail(ZK_ERR_INVALID, "%s: null pointer", who);
  if (!(eps >= 0.0f)) return fail(ZK_ERR_INVALID, "%s: eps must be >= 0", who);
  return ZK_OK;
}

extern "C" int zk_layernorm(const void *x, const void *residual,
                            const void *gamma, const void *beta, void *y,
                            int64_t rows, int64_t hidden, float eps, int dtype,
                            void *stream) {
  int st = ln_check("zk_layernorm", x, gamma, beta, y, rows, hidden, eps);
  if (st || rows == 0) return st;
  hipStream_t s = as_stream(stream);
  if (dtype == ZK_F32)
    return ln_impl<float, false>(x, residual, gamma, beta, y, nullptr, 1.f, rows, hidden, eps, s);
  if (dtype == ZK_F16)
    return ln_impl<f16, false>(x, residual, gamma, beta, y, nullptr, 1.f, rows, hidden, eps, s);
  return fail(ZK_ERR_UNSUPPORTED, "zk_layernorm: dtype %d not supported", dtype);
}

extern "C" int zk_layernorm_q8(const void *x, const void *residual, const void *gamma,
                               const void *beta, void *y, int8_t *q, int64_t rows,
                               int64_t hidden, float eps, float q_scale, void *stream) {
  int st = ln_check("zk_layernorm_q8", x, gamma, beta, y, rows, hidden, eps);
  if (st || rows == 0) return st;
  if (!q) return fail(ZK_ERR_INVALID, "zk_layernorm_q8: null pointer");
  if (!(q_scale > 0.f)) return fail(ZK_ERR_INVALID, "zk_layernorm_q8: q_scale must be > 0");
  return ln_impl<f16, true>(x, residual, gamma, beta, y, q, q_scale, rows, hidden, eps,
                            as_stream(stream));
}

extern "C" int zk_layernorm_q8_res_ln(const void *x, const void *residual, const float *res_ln,
                                      const void *res_gamma, const void *res_beta,
                                      const void *gamma, const void *beta, void *y, int8_t *q,
                                      int64_t rows, int64_t hidden, float eps, float q_scale,
                                      void *stream) {
  const char *who = "zk_layernorm_q8_res_ln";
  int st = ln_check(who, x, gamma, beta, y, rows, hidden, eps);
  if (st || rows == 0) return st;
  if (!q || !residual || !res_ln || !res_gamma || !res_beta)
    return fail(ZK_ERR_INVALID, "%s: null pointer", who);
  if (!(q_scale > 0.f)) return fail(ZK_ERR_INVALID, "%s: q_scale must be > 0", who);
  if (!aligned8(res_ln)) return fail(ZK_ERR_UNSUPPORTED, "%s: res_ln must be 8-byte aligned", who);
  return ln_impl<f16, true>(x, residual, gamma, beta, y, q, q_scale, rows, hidden, eps,
                            as_stream(stream), false,
                            ResLn<f16>{(const float2 *)res_ln, (const f16 *)res_gamma,
                                       (const f16 *)res_beta});
}

extern "C" int zk_layernorm_add(const void *x, const void *residual, const void *gamma,
                                const void *beta, void *y, int64_t rows, int64_t hidden,
                                float eps, int dtype, void *stream) {
  int st = ln_check("zk_layernorm_add", x, gamma, beta, y, rows, hidden, eps);
  if (st || rows == 0) return st;
  if (!residual) return fail(ZK_ERR_INVALID, "zk_layernorm_add: null residual");
  hipStream_t s = as_stream(stream);
  if (dtype == ZK_F32)
    return ln_impl<float, false>(x, residual, gamma, beta, y, nullptr, 1.f, rows, hidden, eps, s,
                                 true);
  if (dtype == ZK_F16)
    return ln_impl<f16, false>(x, residual, gamma, beta, y, nullptr, 1.f, rows, hidden, eps, s,
                               true);
  return fail(ZK_ERR_UNSUPPORTED, "zk_layernorm_add: dtype %d not supported", dtype);
}

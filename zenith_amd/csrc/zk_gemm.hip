// GEMMs for gfx950.
//
// zk_gemm_f16 / zk_gemm_i8: MFMA main loop shared by the fp16 and int8
// paths. Both operands are K-major in memory (A[M,K], W[N,K]); each
// workgroup owns a BM x BN output tile, 4 wavefronts in a 2 x 2 grid own
// (BM/2) x (BN/2) sub-tiles built from 32x32 MFMA blocks. K is walked in
// BKB-byte slices staged through two LDS buffers (one barrier per slice);
// the next slice's 16-byte global loads are in flight while the current one
// is multiplied. LDS rows are padded by 16 bytes so the row-strided 16-byte
// fragment reads of a wavefront hit distinct banks. The epilogue (bias,
// GELU, residual, int8 dequantisation) is applied to the accumulators before
// the single store of C.
//
// The B[K,N] (n-contiguous) layout of wmma_matmul is served by transposing B
// once (zk_transpose_f16) into a caller-provided buffer; the Python layer
// does that, so the kernel itself only ever reads K-major operands.
//
// zk_gemm_f32: fp32 SIMT kernel (64x64 tiles, 4x4 outputs per thread) for
// the reference's fp32 `matmul` entry point, which must stay exact fp32.
#include <type_traits>

#include "zk_common.hpp"

namespace zk {

struct GemmParams {
  const void *A;
  const void *B;
  void *C;
  int M, N, K;
  int64_t lda, ldb, ldc;
  const void *bias;
  const void *res;
  int64_t ldr;
  float s_x;
  const float *s_w;
  int tiles_n;
};

struct F16Op {
  typedef f16x8 Frag;
  typedef f32x16 Acc;
  static constexpr int kElem = 2;
  static __device__ __forceinline__ Acc mma(Frag a, Frag b, Acc c) {
    return mfma32x32x16(a, b, c);
  }
};
struct I8Op {
  typedef i32x4 Frag;
  typedef i32x16 Acc;
  static constexpr int kElem = 1;
  static __device__ __forceinline__ Acc mma(Frag a, Frag b, Acc c) {
    return mfma32x32x32_i8(a, b, c);
  }
};

template <typename T> __device__ __forceinline__ float to_f(T v) { return (float)v; }

template <int EPI>
__device__ __forceinline__ float epilogue(float v, float bias, float res) {
  if (EPI == ZK_EPI_NONE) return v;
  v += bias;
  if (EPI == ZK_EPI_BIAS_GELU_ERF) return gelu_erf(v);
  if (EPI == ZK_EPI_BIAS_GELU_TANH) return gelu_tanh(v);
  if (EPI == ZK_EPI_BIAS_RELU) return v > 0.f ? v : 0.f;
  if (EPI == ZK_EPI_BIAS_RESIDUAL) return v + res;
  return v;
}

// Workgroup -> tile. The hardware deals workgroups round-robin over the 8
// XCDs; renumbering so that each XCD receives a contiguous run of tiles
// (same A rows, all N tiles) keeps that run's A and B slices in the XCD's
// own L2.
__device__ __forceinline__ int xcd_tile(int wg, int nwg) {
  if ((nwg & 7) != 0) return wg;
  return (wg & 7) * (nwg >> 3) + (wg >> 3);
}

template <class OP, int BM, int BN, int BKB, int EPI, typename OutT, bool DEQ>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(GemmParams p) {
  constexpr int NT = 256;
  constexpr int WTM = BM / 2, WTN = BN / 2;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int LDB = BKB + 16;  // padded LDS row, bytes
  constexpr int VPR = BKB / 16;  // 16-byte vectors per tile row
  constexpr int VA = BM * VPR / NT, VB = BN * VPR / NT;
  static_assert(BM * VPR % NT == 0 && BN * VPR % NT == 0, "tile/thread mismatch");
  constexpr int STAGE = (BM + BN) * LDB;
  __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int t = xcd_tile(blockIdx.x, gridDim.x);
  const int tm = t / p.tiles_n, tn = t % p.tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int64_t kbytes = (int64_t)p.K * OP::kElem;

  const char *Ab = (const char *)p.A;
  const char *Bb = (const char *)p.B;
  const int64_t lda_b = p.lda * OP::kElem, ldb_b = p.ldb * OP::kElem;

  i32x4 ra[VA], rb[VB];
  auto load = [&](int64_t kb) {
#pragma unroll
    for (int v = 0; v < VA; ++v) {
      const int idx = tid + v * NT, row = idx / VPR, cv = idx % VPR;
      const int64_t kk = kb + cv * 16;
      const int gr = m0 + row;
      ra[v] = (gr < p.M && kk < kbytes)
                  ? *(const i32x4 *)(Ab + (int64_t)gr * lda_b + kk)
                  : i32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int v = 0; v < VB; ++v) {
      const int idx = tid + v * NT, row = idx / VPR, cv = idx % VPR;
      const int64_t kk = kb + cv * 16;
      const int gr = n0 + row;
      rb[v] = (gr < p.N && kk < kbytes)
                  ? *(const i32x4 *)(Bb + (int64_t)gr * ldb_b + kk)
                  : i32x4{0, 0, 0, 0};
    }
  };
  auto stash = [&](int stage) {
    char *As = smem + stage * STAGE, *Bs = As + BM * LDB;
#pragma unroll
    for (int v = 0; v < VA; ++v) {
      const int idx = tid + v * NT, row = idx / VPR, cv = idx % VPR;
      *(i32x4 *)(As + row * LDB + cv * 16) = ra[v];
    }
#pragma unroll
    for (int v = 0; v < VB; ++v) {
      const int idx = tid + v * NT, row = idx / VPR, cv = idx % VPR;
      *(i32x4 *)(Bs + row * LDB + cv * 16) = rb[v];
    }
  };

  typename OP::Acc acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int nk = (int)((kbytes + BKB - 1) / BKB);
  load(0);
  stash(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load((int64_t)(kt + 1) * BKB);
    const char *As = smem + cur * STAGE, *Bs = As + BM * LDB;
#pragma unroll
    for (int ks = 0; ks < BKB; ks += 32) {
      typename OP::Frag a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        a[i] = *(const typename OP::Frag *)(As + (wm * WTM + i * 32 + (lane & 31)) * LDB +
                                            ks + (lane >> 5) * 16);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        b[j] = *(const typename OP::Frag *)(Bs + (wn * WTN + j * 32 + (lane & 31)) * LDB +
                                            ks + (lane >> 5) * 16);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = OP::mma(a[i], b[j], acc[i][j]);
    }
    if (kt + 1 < nk) stash(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: lane owns column (lane % 32) of each 32x32 block and rows
  // 8*(r/4) + 4*(lane/32) + r%4.
  OutT *C = (OutT *)p.C;
  const OutT *bias = (const OutT *)p.bias;
  const OutT *res = (const OutT *)p.res;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int col = n0 + wn * WTN + j * 32 + (lane & 31);
    if (col >= p.N) continue;
    const float b = (EPI != ZK_EPI_NONE) ? to_f(bias[col]) : 0.f;
    const float sc = DEQ ? p.s_x * p.s_w[col] : 1.f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * WTM + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (row < p.M) {
          if constexpr (std::is_same<OutT, int32_t>::value) {
            C[(int64_t)row * p.ldc + col] = acc[i][j][r];  // raw, bit-exact
          } else {
            float v = DEQ ? (float)acc[i][j][r] * sc : (float)acc[i][j][r];
            const float rv = (EPI == ZK_EPI_BIAS_RESIDUAL) ? to_f(res[(int64_t)row * p.ldr + col]) : 0.f;
            C[(int64_t)row * p.ldc + col] = (OutT)epilogue<EPI>(v, b, rv);
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------ dispatch ----
template <class OP, int BM, int BN, int BKB, typename OutT, bool DEQ>
static void launch_epi(const GemmParams &p, int epi, int grid, hipStream_t s) {
  switch (epi) {
    case ZK_EPI_NONE:
      gemm_mfma_kernel<OP, BM, BN, BKB, ZK_EPI_NONE, OutT, DEQ><<<grid, 256, 0, s>>>(p); break;
    case ZK_EPI_BIAS:
      gemm_mfma_kernel<OP, BM, BN, BKB, ZK_EPI_BIAS, OutT, DEQ><<<grid, 256, 0, s>>>(p); break;
    case ZK_EPI_BIAS_GELU_ERF:
      gemm_mfma_kernel<OP, BM, BN, BKB, ZK_EPI_BIAS_GELU_ERF, OutT, DEQ><<<grid, 256, 0, s>>>(p); break;
    case ZK_EPI_BIAS_GELU_TANH:
      gemm_mfma_kernel<OP, BM, BN, BKB, ZK_EPI_BIAS_GELU_TANH, OutT, DEQ><<<grid, 256, 0, s>>>(p); break;
    case ZK_EPI_BIAS_RESIDUAL:
      gemm_mfma_kernel<OP, BM, BN, BKB, ZK_EPI_BIAS_RESIDUAL, OutT, DEQ><<<grid, 256, 0, s>>>(p); break;
    case ZK_EPI_BIAS_RELU:
      gemm_mfma_kernel<OP, BM, BN, BKB, ZK_EPI_BIAS_RELU, OutT, DEQ><<<grid, 256, 0, s>>>(p); break;
  }
}

template <class OP, typename OutT, bool DEQ>
static void launch_mfma(GemmParams p, int epi, hipStream_t s) {
  constexpr int BKB = 128;
  // Tile choice: 128x128 unless that leaves most of the 256 CUs idle, then
  // 64-row tiles to double the workgroup count.
  const int64_t t128 = (int64_t)((p.M + 127) / 128) * ((p.N + 127) / 128);
  if (t128 >= 256) {
    p.tiles_n = (p.N + 127) / 128;
    launch_epi<OP, 128, 128, BKB, OutT, DEQ>(p, epi, (int)t128, s);
  } else {
    p.tiles_n = (p.N + 127) / 128;
    const int grid = ((p.M + 63) / 64) * p.tiles_n;
    launch_epi<OP, 64, 128, BKB, OutT, DEQ>(p, epi, grid, s);
  }
}

// ------------------------------------------------------------- fp32 SIMT --
template <bool TRANS_B>
__global__ __launch_bounds__(256) void gemm_f32_kernel(
    const float *__restrict__ A, const float *__restrict__ B,
    float *__restrict__ C, int M, int N, int K, int64_t lda, int64_t ldb,
    int64_t ldc) {
  __shared__ float As[16][64 + 4];
  __shared__ float Bs[16][64 + 4];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    // A tile: 64 rows x 16 k, k fastest across lanes
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int idx = tid + v * 256, r = idx >> 4, k = idx & 15;
      const int gr = m0 + r, gk = k0 + k;
      As[k][r] = (gr < M && gk < K) ? A[(int64_t)gr * lda + gk] : 0.f;
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int idx = tid + v * 256;
      if (TRANS_B) {  // W[N,K]: k fastest
        const int c = idx >> 4, k = idx & 15, gc = n0 + c, gk = k0 + k;
        Bs[k][c] = (gc < N && gk < K) ? B[(int64_t)gc * ldb + gk] : 0.f;
      } else {  // B[K,N]: n fastest
        const int k = idx >> 6, c = idx & 63, gc = n0 + c, gk = k0 + k;
        Bs[k][c] = (gc < N && gk < K) ? B[(int64_t)gk * ldb + gc] : 0.f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[k][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[k][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = m0 + ty * 4 + i;
    if (r >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = n0 + tx * 4 + j;
      if (c < N) C[(int64_t)r * ldc + c] = acc[i][j];
    }
  }
}

static int check_dims(const char *who, int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N < 0 || K < 0) return fail(ZK_ERR_INVALID, "%s: negative size", who);
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff)
    return fail(ZK_ERR_UNSUPPORTED, "%s: dimension exceeds int32", who);
  return ZK_OK;
}

}  // namespace zk

using namespace zk;

extern "C" int zk_gemm_f16(const void *A, const void *B, void *C, int64_t M,
                           int64_t N, int64_t K, int64_t lda, int64_t ldb,
                           int64_t ldc, int trans_b, int out_dtype,
                           const void *bias, const void *residual, int64_t ldr,
                           int epilogue, void *stream) {
  int st = check_dims("zk_gemm_f16", M, N, K);
  if (st) return st;
  if (M == 0 || N == 0) return ZK_OK;
  if (!A || !B || !C) return fail(ZK_ERR_INVALID, "zk_gemm_f16: null pointer");
  if (epilogue < ZK_EPI_NONE || epilogue > ZK_EPI_BIAS_RELU)
    return fail(ZK_ERR_INVALID, "zk_gemm_f16: bad epilogue %d", epilogue);
  if (epilogue != ZK_EPI_NONE && !bias)
    return fail(ZK_ERR_INVALID, "zk_gemm_f16: epilogue needs a bias");
  if (epilogue == ZK_EPI_BIAS_RESIDUAL && (!residual || ldr < N))
    return fail(ZK_ERR_INVALID, "zk_gemm_f16: residual epilogue needs residual and ldr >= N");
  if (!trans_b)
    return fail(ZK_ERR_UNSUPPORTED,
                "zk_gemm_f16: B[K,N] operand must be transposed to W[N,K] first "
                "(zk_transpose_f16)");
  if (lda < K || ldb < K || ldc < N)
    return fail(ZK_ERR_INVALID, "zk_gemm_f16: leading dimension too small");
  if (K % 8 || lda % 8 || ldb % 8 || !aligned16(A) || !aligned16(B))
    return fail(ZK_ERR_UNSUPPORTED,
                "zk_gemm_f16: K, lda, ldb must be multiples of 8 and A, B 16-byte aligned");
  if (out_dtype != ZK_F16 && out_dtype != ZK_F32)
    return fail(ZK_ERR_UNSUPPORTED, "zk_gemm_f16: out_dtype %d not supported", out_dtype);
  if (K == 0) return fail(ZK_ERR_UNSUPPORTED, "zk_gemm_f16: K == 0");
  GemmParams p{A, B, C, (int)M, (int)N, (int)K, lda, ldb, ldc, bias, residual, ldr, 1.f, nullptr, 0};
  hipStream_t s = as_stream(stream);
  if (out_dtype == ZK_F16) launch_mfma<F16Op, f16, false>(p, epilogue, s);
  else launch_mfma<F16Op, float, false>(p, epilogue, s);
  return check_launch("zk_gemm_f16");
}

extern "C" int zk_gemm_i8(const int8_t *A, const int8_t *W, void *C, int64_t M,
                          int64_t N, int64_t K, int64_t lda, int64_t ldw,
                          int64_t ldc, float s_x, const float *s_w,
                          const void *bias, const void *residual, int64_t ldr,
                          int epilogue, int out_dtype, void *stream) {
  int st = check_dims("zk_gemm_i8", M, N, K);
  if (st) return st;
  if (M == 0 || N == 0) return ZK_OK;
  if (!A || !W || !C) return fail(ZK_ERR_INVALID, "zk_gemm_i8: null pointer");
  if (epilogue < ZK_EPI_NONE || epilogue > ZK_EPI_BIAS_RELU)
    return fail(ZK_ERR_INVALID, "zk_gemm_i8: bad epilogue %d", epilogue);
  if (lda < K || ldw < K || ldc < N)
    return fail(ZK_ERR_INVALID, "zk_gemm_i8: leading dimension too small");
  if (K % 16 || lda % 16 || ldw % 16 || !aligned16(A) || !aligned16(W))
    return fail(ZK_ERR_UNSUPPORTED,
                "zk_gemm_i8: K, lda, ldw must be multiples of 16 and A, W 16-byte aligned");
  if (K == 0) return fail(ZK_ERR_UNSUPPORTED, "zk_gemm_i8: K == 0");
  if (K > 131072)
    return fail(ZK_ERR_UNSUPPORTED, "zk_gemm_i8: K > 131072 could overflow int32 accumulators");
  hipStream_t s = as_stream(stream);
  GemmParams p{A, W, C, (int)M, (int)N, (int)K, lda, ldw, ldc, bias, residual, ldr, s_x, s_w, 0};
  if (out_dtype == ZK_I32) {
    if (epilogue != ZK_EPI_NONE)
      return fail(ZK_ERR_INVALID, "zk_gemm_i8: int32 output takes no epilogue");
    launch_mfma<I8Op, int32_t, false>(p, ZK_EPI_NONE, s);
    return check_launch("zk_gemm_i8");
  }
  if (!s_w) return fail(ZK_ERR_INVALID, "zk_gemm_i8: dequantised output needs s_w");
  if (!(s_x > 0.f)) return fail(ZK_ERR_INVALID, "zk_gemm_i8: s_x must be > 0");
  if (epilogue != ZK_EPI_NONE && !bias)
    return fail(ZK_ERR_INVALID, "zk_gemm_i8: epilogue needs a bias");
  if (epilogue == ZK_EPI_BIAS_RESIDUAL && (!residual || ldr < N))
    return fail(ZK_ERR_INVALID, "zk_gemm_i8: residual epilogue needs residual and ldr >= N");
  if (out_dtype == ZK_F16) launch_mfma<I8Op, f16, true>(p, epilogue, s);
  else if (out_dtype == ZK_F32) launch_mfma<I8Op, float, true>(p, epilogue, s);
  else return fail(ZK_ERR_UNSUPPORTED, "zk_gemm_i8: out_dtype %d not supported", out_dtype);
  return check_launch("zk_gemm_i8");
}

extern "C" int zk_gemm_f32(const float *A, const float *B, float *C, int64_t M,
                           int64_t N, int64_t K, int64_t lda, int64_t ldb,
                           int64_t ldc, int trans_b, void *stream) {
  int st = check_dims("zk_gemm_f32", M, N, K);
  if (st) return st;
  if (M == 0 || N == 0) return ZK_OK;
  if (!A || !B || !C) return fail(ZK_ERR_INVALID, "zk_gemm_f32: null pointer");
  if (lda < K || ldc < N || (trans_b ? ldb < K : ldb < N))
    return fail(ZK_ERR_INVALID, "zk_gemm_f32: leading dimension too small");
  if ((M + 63) / 64 > 65535) return fail(ZK_ERR_UNSUPPORTED, "zk_gemm_f32: M too large");
  dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
  hipStream_t s = as_stream(stream);
  if (trans_b)
    gemm_f32_kernel<true><<<grid, 256, 0, s>>>(A, B, C, (int)M, (int)N, (int)K, lda, ldb, ldc);
  else
    gemm_f32_kernel<false><<<grid, 256, 0, s>>>(A, B, C, (int)M, (int)N, (int)K, lda, ldb, ldc);
  return check_launch("zk_gemm_f32");
}

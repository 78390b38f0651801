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
#include <stdlib.h>

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

// LDS tiles hold 128-byte K slices of BM (A) and BN (B) rows, unpadded; the
// 16-byte chunk c of row r lives at chunk position c ^ (r & 7), so the 8 rows
// a fragment read touches at one k fall on 8 different bank groups.
__device__ __forceinline__ int swz(int row, int chunk) {
  return row * 128 + ((chunk ^ (row & 7)) << 4);
}

template <int BM, int BN>
struct EpiTile {
  static constexpr int ROWS = BM < 128 ? BM : 128;  // rows staged per pass
  static constexpr int PITCH = BN + 8;                // fp32 words per LDS row
  static constexpr int BYTES = ROWS * PITCH * 4;
};

template <class OP, int BM, int BN, int WM, int WN>
struct GemmCfg {
  static constexpr int NT = WM * WN * 64;
  static constexpr int BKB = 128;  // bytes of K per stage
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int VA = BM * 8 / NT, VB = BN * 8 / NT;
  static constexpr int STAGE = (BM + BN) * BKB;
  static constexpr int SMEM = (2 * STAGE > EpiTile<BM, BN>::BYTES) ? 2 * STAGE : EpiTile<BM, BN>::BYTES;
  static_assert(BM * 8 % NT == 0 && BN * 8 % NT == 0, "tile/thread mismatch");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be 32-aligned");
  static_assert(EpiTile<BM, BN>::ROWS % WTM == 0 || WTM % EpiTile<BM, BN>::ROWS == 0, "epilogue pass");
};

// Two waves per SIMD: the register budget (256 per lane) holds the two
// prefetch register sets, the fragments and the accumulators without spills.
template <class OP, int BM, int BN, int WM, int WN, int EPI, typename OutT, bool DEQ>
__global__ __launch_bounds__(WM * WN * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_mfma_kernel(GemmParams p) {
  typedef GemmCfg<OP, BM, BN, WM, WN> G;
  constexpr int NT = G::NT, BKB = G::BKB, TM = G::TM, TN = G::TN;
  constexpr int WTM = G::WTM, WTN = G::WTN, VA = G::VA, VB = G::VB;
  __shared__ __attribute__((aligned(16))) char smem[G::SMEM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int t = xcd_tile(blockIdx.x, gridDim.x);
  const int tm = t / p.tiles_n, tn = t % p.tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int64_t kbytes = (int64_t)p.K * OP::kElem;
  // Raw buffer descriptors over this workgroup's A rows [m0, m0 + BM) and
  // B rows [n0, n0 + BN): a load whose offset falls past the last valid row
  // returns 0 in hardware, so edge tiles need no branches. K-tail chunks
  // (k >= K inside a row) are redirected to an out-of-range offset.
  const int64_t lda_b = p.lda * OP::kElem, ldb_b = p.ldb * OP::kElem;
  const int a_rows = min(BM, p.M - m0), b_rows = min(BN, p.N - n0);
  const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
      (void *)((const char *)p.A + (int64_t)m0 * lda_b), (short)0,
      (int)((a_rows - 1) * lda_b + kbytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
      (void *)((const char *)p.B + (int64_t)n0 * ldb_b), (short)0,
      (int)((b_rows - 1) * ldb_b + kbytes), 0x00020000);
  constexpr int OOB = 0x7ffffff0;
  // thread -> (row = tid / 8 + v * NT / 8, 16-byte chunk = tid % 8): eight
  // consecutive threads read one 128-byte row segment.
  const int crow = tid >> 3, cchunk = (tid & 7) << 4;
  const int a_off0 = (int)(crow * lda_b) + cchunk, a_step = (int)((NT / 8) * lda_b);
  const int b_off0 = (int)(crow * ldb_b) + cchunk, b_step = (int)((NT / 8) * ldb_b);

  const int kbytes32 = (int)kbytes;
  auto load = [&](int kb, i32x4 (&ra)[VA], i32x4 (&rb)[VB]) {
    const bool kin = kb + cchunk < kbytes32;
#pragma unroll
    for (int v = 0; v < VA; ++v)
      ra[v] = __builtin_amdgcn_raw_buffer_load_b128(rA, kin ? a_off0 + v * a_step + kb : OOB, 0, 0);
#pragma unroll
    for (int v = 0; v < VB; ++v)
      rb[v] = __builtin_amdgcn_raw_buffer_load_b128(rB, kin ? b_off0 + v * b_step + kb : OOB, 0, 0);
  };
  auto stash = [&](int stage, const i32x4 (&ra)[VA], const i32x4 (&rb)[VB]) {
    char *As = smem + stage * G::STAGE, *Bs = As + BM * BKB;
#pragma unroll
    for (int v = 0; v < VA; ++v) {
      const int idx = tid + v * NT;
      *(i32x4 *)(As + swz(idx >> 3, idx & 7)) = ra[v];
    }
#pragma unroll
    for (int v = 0; v < VB; ++v) {
      const int idx = tid + v * NT;
      *(i32x4 *)(Bs + swz(idx >> 3, idx & 7)) = rb[v];
    }
  };

  typename OP::Acc acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  // Fragments are double-buffered in registers: the reads for k-step ks+1
  // are issued before the MFMAs of k-step ks.
  constexpr int KS = BKB / 32;
  auto compute = [&](int stage) {
    const char *As = smem + stage * G::STAGE, *Bs = As + BM * BKB;
    typename OP::Frag a[2][TM], b[2][TN];
    auto rd = [&](int ks, typename OP::Frag (&fa)[TM], typename OP::Frag (&fb)[TN]) {
      const int chunk = ks * 2 + (lane >> 5);
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[i] = *(const typename OP::Frag *)(As + swz(wm * WTM + i * 32 + (lane & 31), chunk));
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[j] = *(const typename OP::Frag *)(Bs + swz(wn * WTN + j * 32 + (lane & 31), chunk));
    };
    rd(0, a[0], b[0]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) rd(ks + 1, a[(ks + 1) & 1], b[(ks + 1) & 1]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = OP::mma(a[ks & 1][i], b[ks & 1][j], acc[i][j]);
    }
  };

  // Main loop: K slice kt is staged in LDS[kt % 2]; global loads run two
  // slices ahead in one of two register sets. The steady-state loop is
  // unrolled by two (statically named register sets) and contains no
  // conditional load or stash, so every s_waitcnt in it waits only for the
  // older register set; the last one to three slices are peeled.
  const int nk = (int)((kbytes + BKB - 1) / BKB);
  i32x4 ra0[VA], rb0[VB], ra1[VA], rb1[VB];
  load(0, ra0, rb0);
  if (nk > 1) load(BKB, ra1, rb1);
  stash(0, ra0, rb0);
  __syncthreads();
  int kt = 0;
  // sched_barrier(0) keeps the compiler from sinking the prefetch below the
  // MFMAs (which would shorten the prefetch distance to one slice).
  for (; kt + 3 < nk; kt += 2) {
    load((kt + 2) * BKB, ra0, rb0);
    __builtin_amdgcn_sched_barrier(0);
    compute(0);
    __builtin_amdgcn_sched_barrier(0);
    stash(1, ra1, rb1);
    __syncthreads();
    load((kt + 3) * BKB, ra1, rb1);
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
    __builtin_amdgcn_sched_barrier(0);
    stash(0, ra0, rb0);
    __syncthreads();
  }
  const int rem = nk - kt;  // 1, 2 or 3 slices left; slice kt is in LDS[0]
  if (rem == 3) {
    load((kt + 2) * BKB, ra0, rb0);
    compute(0);
    stash(1, ra1, rb1);
    __syncthreads();
    compute(1);
    stash(0, ra0, rb0);
    __syncthreads();
    compute(0);
  } else if (rem == 2) {
    compute(0);
    stash(1, ra1, rb1);
    __syncthreads();
    compute(1);
  } else {
    compute(0);
  }
  __syncthreads();

  // Epilogue, in passes of EpiTile::ROWS rows: waves write their scaled /
  // biased / activated accumulators into an fp32 LDS tile (lane: column
  // lane % 32, rows 8*(r/4) + 4*(lane/32) + r%4 of each 32x32 block), then
  // all threads stream the tile out as 8-column vectors, adding the residual
  // on the way.
  typedef EpiTile<BM, BN> E;
  float *Cs = (float *)smem;
  OutT *C = (OutT *)p.C;
  const OutT *bias = (const OutT *)p.bias;
  const OutT *res = (const OutT *)p.res;
  const bool vec_ok = (p.ldc % 8 == 0) && aligned16(p.C) &&
                      (EPI != ZK_EPI_BIAS_RESIDUAL || ((p.ldr % 8 == 0) && aligned16(p.res)));
#pragma unroll
  for (int pass = 0; pass < BM / E::ROWS; ++pass) {
    const int prow0 = pass * E::ROWS;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int ncol = wn * WTN + j * 32 + (lane & 31);
      const int col = n0 + ncol;
      float b = 0.f, sc = 1.f;
      if (col < p.N) {
        if (EPI != ZK_EPI_NONE) b = to_f(bias[col]);
        if (DEQ) sc = p.s_x * p.s_w[col];
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int mbase = wm * WTM + i * 32;
        if (mbase < prow0 || mbase >= prow0 + E::ROWS) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int mloc = mbase - prow0 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
          if constexpr (std::is_same<OutT, int32_t>::value) {
            ((int *)Cs)[mloc * E::PITCH + ncol] = acc[i][j][r];
          } else {
            const float v = DEQ ? (float)acc[i][j][r] * sc : (float)acc[i][j][r];
            Cs[mloc * E::PITCH + ncol] = epilogue<EPI == ZK_EPI_BIAS_RESIDUAL ? ZK_EPI_BIAS : EPI>(v, b, 0.f);
          }
        }
      }
    }
    __syncthreads();
    constexpr int GPR = BN / 8;  // 8-column groups per row
    for (int g = tid; g < E::ROWS * GPR; g += NT) {
      const int rl = g / GPR, cl = (g % GPR) * 8;
      const int row = m0 + prow0 + rl, col = n0 + cl;
      if (row >= p.M || col >= p.N) continue;
      const float *src = Cs + rl * E::PITCH + cl;
      OutT *dst = C + (int64_t)row * p.ldc + col;
      if (vec_ok && col + 8 <= p.N) {
        f32x4 lo = *(const f32x4 *)src, hi = *(const f32x4 *)(src + 4);
        if constexpr (std::is_same<OutT, int32_t>::value) {
          *(f32x4 *)dst = lo;  // raw bits of the int32 accumulators
          *(f32x4 *)(dst + 4) = hi;
        } else {
          float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          if constexpr (EPI == ZK_EPI_BIAS_RESIDUAL) {
            const OutT *rp = res + (int64_t)row * p.ldr + col;
            if constexpr (std::is_same<OutT, f16>::value) {
              const f16x8 rv = *(const f16x8 *)rp;
#pragma unroll
              for (int e = 0; e < 8; ++e) v[e] += (float)rv[e];
            } else {
#pragma unroll
              for (int e = 0; e < 8; ++e) v[e] += to_f(rp[e]);
            }
          }
          if constexpr (std::is_same<OutT, f16>::value) {
            f16x8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = (f16)v[e];
            *(f16x8 *)dst = o;
          } else {
            *(f32x4 *)dst = f32x4{v[0], v[1], v[2], v[3]};
            *(f32x4 *)(dst + 4) = f32x4{v[4], v[5], v[6], v[7]};
          }
        }
      } else {
        for (int e = 0; e < 8 && col + e < p.N; ++e) {
          if constexpr (std::is_same<OutT, int32_t>::value) {
            dst[e] = ((const int *)src)[e];
          } else {
            float v = src[e];
            if (EPI == ZK_EPI_BIAS_RESIDUAL) v += to_f(res[(int64_t)row * p.ldr + col + e]);
            dst[e] = (OutT)v;
          }
        }
      }
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------ dispatch ----
template <class OP, int BM, int BN, int WM, int WN, typename OutT, bool DEQ>
static void launch_epi(GemmParams p, int epi, hipStream_t s) {
  p.tiles_n = (p.N + BN - 1) / BN;
  const int grid = ((p.M + BM - 1) / BM) * p.tiles_n;
  constexpr int NT = WM * WN * 64;
#define ZK_L(E) gemm_mfma_kernel<OP, BM, BN, WM, WN, E, OutT, DEQ><<<grid, NT, 0, s>>>(p)
  switch (epi) {
    case ZK_EPI_NONE: ZK_L(ZK_EPI_NONE); break;
    case ZK_EPI_BIAS: ZK_L(ZK_EPI_BIAS); break;
    case ZK_EPI_BIAS_GELU_ERF: ZK_L(ZK_EPI_BIAS_GELU_ERF); break;
    case ZK_EPI_BIAS_GELU_TANH: ZK_L(ZK_EPI_BIAS_GELU_TANH); break;
    case ZK_EPI_BIAS_RESIDUAL: ZK_L(ZK_EPI_BIAS_RESIDUAL); break;
    case ZK_EPI_BIAS_RELU: ZK_L(ZK_EPI_BIAS_RELU); break;
  }
#undef ZK_L
}

// Tile configurations (BM x BN, waves WM x WN; every wave owns 64x64 except
// cfg 3, whose waves own 32x64):
//   0: 128x128, 2x2 (256 threads)    1: 256x128, 4x2 (512 threads)
//   2: 128x256, 2x4 (512 threads)    3:  64x128, 2x2 (256 threads)
static int pick_cfg(int M, int N) {
  static int forced = -2;
  if (forced == -2) {
    const char *e = getenv("ZK_GEMM_CFG");
    forced = e ? atoi(e) : -1;
  }
  if (forced >= 0 && forced <= 3) return forced;
  auto tiles = [&](int bm, int bn) { return (int64_t)((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  if (tiles(256, 128) >= 256) return 1;
  if (tiles(128, 128) >= 192) return 0;
  return 3;
}

template <class OP, typename OutT, bool DEQ>
static void launch_mfma(GemmParams p, int epi, hipStream_t s) {
  switch (pick_cfg(p.M, p.N)) {
    case 0: launch_epi<OP, 128, 128, 2, 2, OutT, DEQ>(p, epi, s); break;
    case 1: launch_epi<OP, 256, 128, 4, 2, OutT, DEQ>(p, epi, s); break;
    case 2: launch_epi<OP, 128, 256, 2, 4, OutT, DEQ>(p, epi, s); break;
    default: launch_epi<OP, 64, 128, 2, 2, OutT, DEQ>(p, epi, s); break;
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

// GEMMs for gfx950.
//
// zk_gemm_f16 / zk_gemm_i8 share one MFMA kernel. Both operands are K-major
// in memory (A[M,K], W[N,K]) and the kernel is byte-generic: an fp16 MFMA
// step (32x32x16 or 16x16x32) and an int8 step (32x32x32 or 16x16x64) read
// the same 16 bytes per lane and operand, so one LDS layout serves both.
//
// Workgroup: 4 wavefronts in a 2 x 2 grid or 8 in a 2 x 4 / 4 x 2 grid,
// each owning a (BM/WM) x (BN/WN) wave tile made of MS x MS MFMA blocks
// (MS = 32 or 16). The macro tile is chosen per shape from measurements
// (pick_cfg): 8-wave 256-row tiles (two waves of one workgroup per SIMD)
// where the grid still fills the chip, small tiles with several workgroups
// per CU for the narrow projections.
//
// K is walked in slices of BKB bytes per row. A slice of A and W goes from
// global memory straight into LDS with buffer_load ... lds (16 bytes per
// lane, 1 KB per wavefront instruction, no VGPR staging), into a ring of
// ST stages; slices are issued ST-1 ahead, and each iteration has exactly
// one barrier, preceded by an explicit vmcnt wait that leaves the younger
// slices in flight. Rows are addressed through raw buffer descriptors that
// end at the last valid row, so loads past M / N return zeros; chunks past
// K are redirected out of range.
//
// LDS rows hold BKB bytes as 16-byte chunks; chunk c of row r sits at slot
// c ^ f(r), with f spreading the 16 rows one fragment read touches over
// 16 distinct 16-byte bank groups (a 256-byte bank period holds 2 rows of
// 128 bytes or 4 rows of 64 bytes).
//
// Epilogue: each wavefront stages one MS-row stripe of its wave tile in
// LDS as fp32 (after scale / bias / activation), then streams it out as
// 8-column vectors, adding the residual on the way; no workgroup barrier is
// needed between stripes.
//
// The B[K,N] (n-contiguous) layout of wmma_matmul is served by transposing B
// once (zk_transpose_f16) into a caller-provided buffer; the Python layer
// does that, so the kernel itself only ever reads K-major operands.
//
// zk_gemm_f32: fp32 SIMT kernel (64x64 tiles, 4x4 outputs per thread) for
// the reference's fp32 `matmul` entry point, which must stay exact fp32.
#include <stdlib.h>

#include <type_traits>

#include "zk_attn_tile.hpp"

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
  int tiles_m;
  int group_m;
  float s_q;  // int8 output: scale of the re-quantisation
  // split-K: workgroup (tile t, split s) = blockIdx t * splits + s covers K
  // slices [s * nk_per, +nk_per) and writes its fp32 partial tile to
  // C + s * split_stride (C is then the workspace, ldc = N)
  int splits;
  int nk_per;
  int64_t split_stride;
  // fused QKV projection + attention (kEpiQkvAttn): sequences of `seq`
  // rows, `batch` of them, key-padding lengths, softmax scale * log2(e)
  int seq;
  int batch;
  const int32_t *valid_lens;
  float scale_log2;
  // LayerNorm of the A rows folded into the GEMM (kEpiLnIn*, and the fused
  // attention when ln_part is set): A holds the LN input x, the weight is
  // gamma-scaled (W'[n,k] = W[n,k] gamma[k]) and the epilogue forms
  //   rstd[m] (acc - mean[m] ln_s[n]) + ln_c[n],
  // ln_s = column sums of W', ln_c = beta . W^T + bias. mean / rstd come from
  // the per-row partial statistics ln_part [M][ln_nparts] of (mean, M2) over
  // kLnSeg-column segments; tile column 0 writes them to ln_out [M] if set.
  const float *ln_part;
  int ln_nparts;
  float ln_eps;
  const float *ln_s;
  const float *ln_c;
  float *ln_out;
  // kEpiResStats: the residual is LN(res) with res_ln [M] (mean, rstd) and
  // fp16 res_gamma / res_beta when res_ln is set; the fp16-rounded outputs'
  // per-row (mean, M2) over kLnSeg-column segments go to part_out
  // [M][N / kLnSeg].
  const float *res_ln;
  const void *res_gamma;
  const void *res_beta;
  float *part_out;
  // Fragment order, the layout of an fp16 MFMA operand of 32 rows: for row
  // block rb (rows 32 rb .. +31) and k-step ks (columns 16 ks .. +15) of an
  // R x K matrix, the 1 KB at byte (rb * K / 16 + ks) * 1024 holds lane l's
  // 16 bytes, X[32 rb + l % 32][16 ks + 8 (l / 32) .. +7], at byte 16 l.
  // a_pk: A in fragment order (kernels instantiated with APK, K a multiple
  // of 64; lda unused): each fragment is one 1 KB DMA into LDS.
  // c_pk: C written in fragment order (kEpiLnInGelu; ldc unused).
  const void *a_pk;
  int c_pk;
};

// Internal epilogues (not public ZK_EPI_* values): the fused QKV projection +
// attention; bias + residual (optionally LayerNorm-ed on the fly) with
// per-row partial statistics of the output; and the folded LayerNorm of the
// input rows, without or with erf-GELU.
constexpr int kEpiQkvAttn = 100;
constexpr int kEpiResStats = 101;
constexpr int kEpiLnIn = 102;
constexpr int kEpiLnInGelu = 103;

// Row statistics travel as (mean, M2) partials of kLnSeg-column segments
// (the 96-column wave tiles of the producing GEMM); a consumer holds at most
// kLnMaxParts of them per row in registers (rows of up to 1536 values).
constexpr int kLnSeg = 96;
constexpr int kLnMaxParts = 16;

// (mean, rstd) of a row of nparts x kLnSeg values from its partial
// (mean, M2) pairs (Chan et al.'s pairwise update for equal counts, in a
// fixed order).
__device__ __forceinline__ float2 ln_merge(const float2 (&pr)[kLnMaxParts], int nparts,
                                           float eps) {
  float sm = 0.f;
#pragma unroll
  for (int q = 0; q < kLnMaxParts; ++q)
    if (q < nparts) sm += pr[q].x;
  const float mean = sm / (float)nparts;
  float m2 = 0.f, dev = 0.f;
#pragma unroll
  for (int q = 0; q < kLnMaxParts; ++q)
    if (q < nparts) {
      const float d = pr[q].x - mean;
      m2 += pr[q].y;
      dev = fmaf(d, d, dev);
    }
  const float var = fmaf((float)kLnSeg, dev, m2) / ((float)kLnSeg * (float)nparts);
  return make_float2(mean, 1.0f / sqrtf(var + eps));
}

// MFMA step on 16 bytes per lane and operand. MS = 32: lane l supplies row
// l % 32, bytes [16 * (l / 32), +16) of the 32-byte k-step; the result
// register r of lane l is D[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32].
// MS = 16: lane l supplies row l % 16, bytes [16 * (l / 16), +16) of the
// 64-byte k-step; register r is D[4 * (l / 16) + r][l % 16].
template <int MS> struct F16Mma;
template <> struct F16Mma<32> {
  typedef f32x16 Acc;
  static constexpr int R = 16;
  static __device__ __forceinline__ Acc mma(f16x8 a, f16x8 b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct F16Mma<16> {
  typedef f32x4 Acc;
  static constexpr int R = 4;
  static __device__ __forceinline__ Acc mma(f16x8 a, f16x8 b, Acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <int MS> struct I8Mma;
template <> struct I8Mma<32> {
  typedef i32x16 Acc;
  static constexpr int R = 16;
  static __device__ __forceinline__ Acc mma(i32x4 a, i32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
};
template <> struct I8Mma<16> {
  typedef i32x4 Acc;
  static constexpr int R = 4;
  static __device__ __forceinline__ Acc mma(i32x4 a, i32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
  }
};

// fp32 on the matrix cores: 16 bytes per lane and operand are four fp32
// values, k0 + 4 * (lane slot) + j, consumed by four chained fp32 MFMAs in
// which element j of every lane is the operand (32x32x2: lane half = k
// index; 16x16x4: lane quarter = k index). The four products together cover
// the same 8 (MS = 32) or 16 (MS = 16) consecutive k as one fp16 step.
template <int MS> struct F32Mma;
template <> struct F32Mma<32> {
  typedef f32x16 Acc;
  static constexpr int R = 16;
  static __device__ __forceinline__ Acc mma(f32x4 a, f32x4 b, Acc c) {
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[0], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[1], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[2], b[2], c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a[3], b[3], c, 0, 0, 0);
  }
};
template <> struct F32Mma<16> {
  typedef f32x4 Acc;
  static constexpr int R = 4;
  static __device__ __forceinline__ Acc mma(f32x4 a, f32x4 b, Acc c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], c, 0, 0, 0);
  }
};

struct F16Op {
  typedef f16x8 Frag;
  template <int MS> using Mma = F16Mma<MS>;
  static constexpr int kElem = 2;
};
struct F32Op {
  typedef f32x4 Frag;
  template <int MS> using Mma = F32Mma<MS>;
  static constexpr int kElem = 4;
};
struct I8Op {
  typedef i32x4 Frag;
  template <int MS> using Mma = I8Mma<MS>;
  static constexpr int kElem = 1;
};

template <typename T> __device__ __forceinline__ float to_f(T v) { return (float)v; }

template <int EPI>
__device__ __forceinline__ float epilogue(float v, float bias) {
  if (EPI == ZK_EPI_NONE) return v;
  v += bias;
  if (EPI == ZK_EPI_BIAS_GELU_ERF) return gelu_erf_fast(v);
  if (EPI == ZK_EPI_BIAS_GELU_TANH) return gelu_tanh_fast(v);
  if (EPI == ZK_EPI_BIAS_RELU) return v > 0.f ? v : 0.f;
  return v;  // BIAS, BIAS_RESIDUAL (residual added at the store)
}

// Workgroup -> (tile_m, tile_n). The hardware deals workgroups round-robin
// over the 8 XCDs; the index is first renumbered so that each XCD receives
// a contiguous run, and the run is then laid out in groups of `group_m`
// tile rows walked column by column, so one XCD's tiles form a compact
// rectangle whose A rows and W rows stay in that XCD's L2.
__device__ __forceinline__ void tile_of(int wg, int nwg, const GemmParams &p, int &tm, int &tn) {
  int t = wg;
  if ((nwg & 7) == 0) t = (wg & 7) * (nwg >> 3) + (wg >> 3);
  const int per_group = p.group_m * p.tiles_n;
  const int first_m = (t / per_group) * p.group_m;
  const int gsz = min(p.tiles_m - first_m, p.group_m);
  const int r = t % per_group;
  tm = first_m + r % gsz;
  tn = r / gsz;
}

template <int BKB>
__device__ __forceinline__ int lds_slot(int row, int c) {
  return BKB == 128 ? (c ^ ((row >> 1) & 7)) : (c ^ ((row >> 2) & 3));
}

constexpr int epi_pitch16(int w) {
  int p = (w + 3) / 4 * 4;
  while (p % 64 != 16 && p % 64 != 48) p += 4;
  return p;
}

template <class OP, int BM, int BN, int MS, int BKB, int ST, int WM = 2, int WN = 2>
struct GemmCfg {
  static constexpr int NW = WM * WN, NT = 64 * NW;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / MS, TN = WTN / MS;
  static constexpr int CH = BKB / 16;          // 16-byte chunks per LDS row
  static constexpr int RPI = 1024 / BKB;       // rows per wavefront DMA instruction
  static constexpr int IA = BM / RPI / NW;     // DMA instructions per wave per slice
  static constexpr int IB = BN / RPI / NW;
  static constexpr int STAGE = (BM + BN) * BKB;
  static constexpr int KCH = MS == 32 ? 2 : 4;  // chunks per MFMA k-step
  static constexpr int KS = CH / KCH;          // MFMA k-steps per slice
  // fp32 words per epilogue LDS row, chosen so one register's worth of
  // writes (32 columns x 2 rows 4 apart for MS = 32; 16 columns x 4
  // consecutive rows for MS = 16) covers 64 distinct banks.
  static constexpr int EPITCH = MS == 32 ? (WTN % 16 == 8 ? WTN : WTN + 8 - WTN % 16 + (WTN % 16 > 8 ? 16 : 0))
                                         : epi_pitch16(WTN);
  static constexpr int EPI_BYTES = NW * MS * EPITCH * 4;
  static constexpr int SMEM = ST * STAGE > EPI_BYTES ? ST * STAGE : EPI_BYTES;
  static_assert(BKB == 64 || BKB == 128, "slice width");
  static_assert(WTM % MS == 0 && WTN % MS == 0, "wave tile must be a multiple of the MFMA block");
  static_assert(BM % (RPI * NW) == 0 && BN % (RPI * NW) == 0, "DMA split");
  static_assert(KS >= 2 && KS % 2 == 0, "k-steps per slice must be even");
  static_assert(ST >= 2 && (ST - 1) * (IA + IB) <= 63, "vmcnt range");
  static_assert(SMEM <= 160 * 1024, "LDS budget");
  static_assert(WTN % 8 == 0, "epilogue vectors");
};

// Scheduling hint for one k-step: NR LDS fragment reads spread evenly over
// NM MFMAs (a read, then its share of MFMAs), so read latency hides under
// matrix work instead of being waited for in front of it.
template <int NR, int NM, int R = 0>
__device__ __forceinline__ void interleave() {
  if constexpr (R < NR) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    __builtin_amdgcn_sched_group_barrier(0x008, NM / NR + (R < NM % NR ? 1 : 0), 0);  // MFMA
    interleave<NR, NM, R + 1>();
  }
}

// Waves per SIMD the register allocation must allow: as many workgroups
// per CU as the LDS ring admits (NW / 4 waves per SIMD each), capped at 3.
constexpr int gemm_waves_per_eu(int smem_bytes, int nw) {
  return nw == 8 ? 2 : smem_bytes <= 53 * 1024 ? 3 : smem_bytes <= 80 * 1024 ? 2 : 1;
}

template <class OP, int BM, int BN, int MS, int BKB, int ST, int WM, int WN, int EPI, typename OutT,
          bool DEQ, bool APK = false>
__global__ __launch_bounds__(64 * WM * WN)
__attribute__((amdgpu_waves_per_eu(gemm_waves_per_eu(GemmCfg<OP, BM, BN, MS, BKB, ST, WM, WN>::SMEM,
                                                     WM * WN))))
void gemm_mfma_kernel(GemmParams p) {
  typedef GemmCfg<OP, BM, BN, MS, BKB, ST, WM, WN> G;
  typedef typename OP::template Mma<MS> MM;
  typedef typename OP::Frag Frag;
  constexpr int TM = G::TM, TN = G::TN, IA = G::IA, IB = G::IB, CH = G::CH;
  constexpr int WTM = G::WTM, WTN = G::WTN, KS = G::KS, KCH = G::KCH, R = MM::R;
  __shared__ __attribute__((aligned(1024))) char smem[G::SMEM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in an SGPR
  const int wm = wave / WN, wn = wave % WN;
  int tm, tn;
  int split = 0, twg = blockIdx.x, nwg = gridDim.x;
  if (p.splits > 1) {
    split = blockIdx.x % p.splits;
    twg = blockIdx.x / p.splits;
    nwg = gridDim.x / p.splits;
  }
  tile_of(twg, nwg, p, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  // Folded LayerNorm: the partial statistics of row m0 + tid are loaded
  // into registers here, so that the loads overlap the main loop; they are
  // merged after it. (Issued after the first slices instead, as the
  // residual below is, they made the encoder 1% slower: a slice wait that
  // does not count them holds until these loads return.)
  constexpr bool LN_ROWS = EPI == kEpiLnIn || EPI == kEpiLnInGelu || EPI == kEpiQkvAttn;
  static_assert(BM <= 64 * WM * WN, "one thread per tile row");
  // Stands in for an absent operand (no statistics, no bias, no lengths) in
  // the unconditional loads below; their values then go unused.
  const void *any = APK ? p.a_pk : p.A;
  float2 ln_pr[LN_ROWS ? kLnMaxParts : 1];
  if constexpr (LN_ROWS) {
    const bool mine = p.ln_part && (int)threadIdx.x < BM && m0 + (int)threadIdx.x < p.M;
    const float2 *src = (const float2 *)p.ln_part + (int64_t)(m0 + threadIdx.x) * p.ln_nparts;
#pragma unroll
    for (int q = 0; q < kLnMaxParts; ++q)
      ln_pr[q] = mine && q < p.ln_nparts ? src[q] : make_float2(0.f, 0.f);
  }
  // The epilogue's per-column constants of this lane's TN columns: bias,
  // dequantisation scale, or the folded LayerNorm's column sums and offsets
  // (col_s: scale, col_c: offset). Loaded here with the row statistics, so
  // that their latency passes under the main loop instead of after the last
  // MFMA.
  constexpr bool LN_COLS = EPI == kEpiLnIn || EPI == kEpiLnInGelu;
  typedef typename std::conditional<std::is_same<OutT, int8_t>::value, f16, OutT>::type BiasT;
  // The raw values are loaded here, unconditionally (column 0 for columns
  // past N), and col_s / col_c formed from them after the main loop: a load
  // under a per-lane condition whose value is converted at once made the
  // wavefront wait for it before requesting its first slice (three to six
  // dependent loads in a row in the bias and dequantisation epilogues:
  // int8 FFN-down + statistics 19.0 -> 18.6 us, encoders 0.8-1.7% faster).
  BiasT col_bias[TN];
  float col_x[TN], col_y[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int col = n0 + wn * WTN + j * MS + lane % MS, cc = col < p.N ? col : 0;
    if constexpr (EPI == kEpiQkvAttn) {  // N is a whole number of 192-column tiles
      const bool ln = p.ln_part != nullptr, bias = p.bias != nullptr;
      col_x[j] = (ln ? p.ln_s : (const float *)any)[ln ? cc : 0];
      col_y[j] = (ln ? p.ln_c : (const float *)any)[ln ? cc : 0];
      col_bias[j] = (bias ? (const BiasT *)p.bias : (const BiasT *)any)[bias ? cc : 0];
    } else {
      if constexpr (EPI != ZK_EPI_NONE && !LN_COLS) col_bias[j] = ((const BiasT *)p.bias)[cc];
      if constexpr (DEQ) col_x[j] = p.s_w[cc];
      if constexpr (LN_COLS) {
        col_x[j] = p.ln_s[cc];
        col_y[j] = p.ln_c[cc];
      }
    }
  }
  float col_s[TN], col_c[TN];
  auto form_cols = [&]() {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + wn * WTN + j * MS + lane % MS;
      col_s[j] = 1.f;
      col_c[j] = 0.f;
      if constexpr (EPI == kEpiQkvAttn) {
        const bool ln = p.ln_part != nullptr;
        col_s[j] = ln ? col_x[j] : 0.f;
        col_c[j] = ln ? col_y[j] : to_f(col_bias[j]);
      } else if (col < p.N) {
        if constexpr (EPI != ZK_EPI_NONE && !LN_COLS) col_c[j] = to_f(col_bias[j]);
        if constexpr (DEQ) col_s[j] = p.s_x * col_x[j];
        if constexpr (LN_COLS) {
          col_s[j] = col_x[j];
          col_c[j] = col_y[j];
        }
      }
    }
  };
  // kEpiResStats: the residual rows of the wave's first stripe (and their
  // LayerNorm statistics) are loaded into registers under the main loop,
  // issued right after the first slices; those of its other stripes right
  // after the main loop, all at once, instead of one dependent load per
  // vector in the epilogue. Every lane loads (out-of-range lanes from the
  // first element), so a stripe is exactly 2 NPV vector loads.
  constexpr int NPV0 = (MS * (WTN / 8) + 63) / 64;
  constexpr bool RES_PREF = EPI == kEpiResStats && std::is_same<OutT, f16>::value && NPV0 <= 6;
  constexpr int NPV = RES_PREF ? NPV0 : 1, NPT = RES_PREF ? G::TM : 1;
  f16x8 res_pv[NPT][NPV];
  float2 res_ms[NPT][NPV];
  auto load_res = [&](int i) {
    const f16 *rb = (const f16 *)p.res;
    const float2 *lb = p.res_ln ? (const float2 *)p.res_ln : (const float2 *)p.res;
#pragma unroll
    for (int k = 0; k < NPV; ++k) {
      const int v = lane + 64 * k, rl = v / (WTN / 8), cl = (v % (WTN / 8)) * 8;
      const int row = m0 + wm * WTM + i * MS + rl, col = n0 + wn * WTN + cl;
      const bool in = v < MS * (WTN / 8) && row < p.M && col + 8 <= p.N;
      // kept whatever `in` is (the epilogue reads only in-range vectors, and
      // res_ms only with res_ln), so that no lane's load is predicated away
      res_pv[i][k] = *(const f16x8 *)(rb + (in ? (int64_t)row * p.ldr + col : 0));
      res_ms[i][k] = lb[in && p.res_ln ? row : 0];
    }
  };
  // With res_ln, the residual LayerNorm's gamma and beta at this lane's
  // vector columns (the same for every stripe of the wave), all loaded
  // before any epilogue store (a load issued after a store could only be
  // waited for together with that store). The fp16 4-wave tiles (one wave
  // per SIMD, registers to spare) load them here, at kernel start, so that
  // their latency passes under the main loop; the others after it.
  constexpr bool EARLY_GB = RES_PREF && WM * WN == 4 && std::is_same<OP, F16Op>::value;
  f16x8 res_g[NPV], res_b[NPV];
  auto load_gb = [&]() {
#pragma unroll
    for (int k = 0; k < NPV; ++k) {
      const int col = n0 + wn * WTN + ((lane + 64 * k) % (WTN / 8)) * 8;
      const int64_t c = col + 8 <= p.N ? col : 0;
      res_g[k] = *(const f16x8 *)((const f16 *)p.res_gamma + c);
      res_b[k] = *(const f16x8 *)((const f16 *)p.res_beta + c);
    }
  };
  if constexpr (EARLY_GB) {
    if (p.res_ln) load_gb();
  }
  // The fused attention's sequence length for this wave's queries, loaded
  // at kernel start for the same reason.
  int attn_len = 0;
  if constexpr (EPI == kEpiQkvAttn) {
    const int b = m0 / p.seq + wave * 32 / p.seq;
    const bool vl = p.valid_lens != nullptr;
    attn_len = (vl ? p.valid_lens : (const int32_t *)any)[vl && b < p.batch ? b : 0];
  }
  const int kbytes = p.K * OP::kElem;
  const int64_t lda_b = p.lda * OP::kElem, ldb_b = p.ldb * OP::kElem;
  const int a_rows = min(BM, p.M - m0), b_rows = min(BN, p.N - n0);
  // APK: the tile's row blocks of the fragment-ordered A, one 1 KB fragment
  // per 32 bytes of a row (kbytes / 32 KB each)
  const int a_blocks = min(BM / 32, (p.M + 31) / 32 - m0 / 32);
  const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
      APK ? (void *)((const char *)p.a_pk + (int64_t)(m0 / 32) * (kbytes / 32) * 1024)
          : (void *)((const char *)p.A + (int64_t)m0 * lda_b),
      (short)0, APK ? a_blocks * (kbytes / 32) * 1024 : (int)((a_rows - 1) * lda_b + kbytes),
      0x00020000);
  const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
      (void *)((const char *)p.B + (int64_t)n0 * ldb_b), (short)0,
      (int)((b_rows - 1) * ldb_b + kbytes), 0x00020000);

  // DMA source offsets. Instruction g of this wave fills tile rows
  // [(wave * I + g) * RPI, +RPI); lane l lands at LDS slot l % CH of row
  // (l / CH) of that group and therefore fetches the logical chunk whose
  // swizzled slot that is.
  // APK: instruction g moves fragment f = wave * IA + g of the slice (row
  // block f / KS, k-step f % KS), 1 KB contiguous, to LDS byte f * 1024 of
  // the stage's A part, where lane l reads its 16 bytes of it back.
  int offA[IA], chA[IA], offB[IB], chB[IB];
#pragma unroll
  for (int g = 0; g < IA; ++g) {
    if constexpr (APK) {
      const int f = wave * IA + g;
      chA[g] = 0;
      offA[g] = ((f / KS) * (kbytes / 32) + f % KS) * 1024 + lane * 16;
    } else {
      const int row = (wave * IA + g) * G::RPI + lane / CH;
      const int c = lds_slot<BKB>(row, lane % CH);  // the swizzle is an involution
      chA[g] = c * 16;
      offA[g] = (int)(row * lda_b) + c * 16;
    }
  }
#pragma unroll
  for (int g = 0; g < IB; ++g) {
    const int row = (wave * IB + g) * G::RPI + lane / CH;
    const int c = lds_slot<BKB>(row, lane % CH);
    chB[g] = c * 16;
    offB[g] = (int)(row * ldb_b) + c * 16;
  }
  typename MM::Acc acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[i][j][r] = 0;

  // Fragment row of this lane inside an MS-row block, and the chunk offset
  // of its half / quarter of the k-step.
  const int frow = lane % MS, fch = lane / MS;
  // Fragments of two consecutive k-steps: k-step ks of every slice uses
  // buffer ks & 1 (KS is even), so the first k-step of the next slice can
  // be read while the last one of this slice is multiplied.
  Frag fa[2][TM], fb[2][TN];
  static_assert(!APK || (MS == 32 && !std::is_same<OP, F32Op>::value), "fragment-ordered A");
  constexpr int PER = IA + IB;  // DMA instructions per slice and wave
  auto rd = [&](int stage, int ks, int buf) {
    const char *As = smem + stage * G::STAGE;
    const char *Bs = As + BM * BKB;
    const int c = ks * KCH + fch;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if constexpr (APK) {
        fa[buf][i] = *(const Frag *)(As + (((wm * WTM + i * MS) / 32) * KS + ks) * 1024 + lane * 16);
      } else {
        const int row = wm * WTM + i * MS + frow;
        fa[buf][i] = *(const Frag *)(As + row * BKB + lds_slot<BKB>(row, c) * 16);
      }
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int row = wn * WTN + j * MS + frow;
      fb[buf][j] = *(const Frag *)(Bs + row * BKB + lds_slot<BKB>(row, c) * 16);
    }
  };
  auto mma_step = [&](int buf) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = MM::mma(fa[buf][i], fb[buf][j], acc[i][j]);
  };

  const int nk_all = (kbytes + BKB - 1) / BKB;
  const int kt0 = p.splits > 1 ? split * p.nk_per : 0;  // first slice of this split
  const int nk = p.splits > 1 ? max(0, min(nk_all - kt0, p.nk_per)) : nk_all;
  // One K slice of A and W: IA + IB wavefront instructions, each moving
  // 1 KB (64 lanes x 16 bytes) into consecutive LDS bytes. The host
  // compilation pass sees an empty statement: its semantic check of this
  // builtin with a run-time offset rejects the kernel, and clang would then
  // silently omit the kernel's launch stub.
#if defined(__HIP_DEVICE_COMPILE__)
#define ZK_ISSUE(kt, stage)                                                                   \
  do {                                                                                        \
    const int kb_ = ((kt) + kt0) * BKB;                                                       \
    char *as_ = smem + (stage) * G::STAGE, *bs_ = as_ + BM * BKB;                             \
    _Pragma("unroll") for (int g = 0; g < IA; ++g)                                            \
        __builtin_amdgcn_raw_ptr_buffer_load_lds(                                             \
            rA, ZK_LDS(as_ + (wave * IA + g) * 1024), 16,                                     \
            kb_ + chA[g] < kbytes ? offA[g] + (APK ? kb_ / BKB * KS * 1024 : kb_)            \
                                  : 0x7ffffff0,                                               \
            0, 0, 0);                                                                         \
    _Pragma("unroll") for (int g = 0; g < IB; ++g)                                            \
        __builtin_amdgcn_raw_ptr_buffer_load_lds(                                             \
            rB, ZK_LDS(bs_ + (wave * IB + g) * 1024), 16,                                     \
            kb_ + chB[g] < kbytes ? offB[g] + kb_ : 0x7ffffff0, 0, 0, 0);                     \
  } while (0)
#else
#define ZK_ISSUE(kt, stage) ((void)(kt), (void)(stage))
#endif
  // res_first: the first stripe's residual rows are requested before the
  // first slice. Loads into registers and DMA loads into LDS complete in
  // order only among their own kind, so a slice wait (at most c loads in
  // flight) guarantees a slice only through the c DMA loads issued after
  // it, and holds for any load into registers still in flight. Issued after
  // the first slices, these loads made the first waits hold until they
  // returned (fp16 encoder 1.6% slower); allowed for as younger loads in
  // those waits, they could have let a wave read a slice before it landed
  // (as loads of A into registers beside the W DMA were seen to do).
  if constexpr (RES_PREF) {
    load_res(0);
    asm volatile("" ::: "memory");
  }
  {
    // Prologue: one slice per stage.
#pragma unroll
    for (int s = 0; s < ST; ++s)
      if (s < nk) ZK_ISSUE(s, s);
    // (the residual rows, loaded into registers before the prologue, are
    // not counted by the slice waits: see res_first)
    wait_slices<ST - 1, PER>(nk - 1);
    lds_barrier();
    rd(0, 0, 0);
    // Main loop over slices. Before the last k-step of slice kt every wave
    // waits for slice kt + 1 and meets at the barrier; by then the ring stage
    // of slice kt has been read completely (its last fragments are in
    // registers), so slice kt + ST is issued into it, and the first
    // fragments of slice kt + 1 are read under the last MFMAs of slice kt.
    auto steps_but_last = [&](int stage) {
#pragma unroll
      for (int ks = 0; ks + 1 < KS; ++ks) {
        rd(stage, ks + 1, (ks + 1) & 1);
        mma_step(ks & 1);
        interleave<TM + TN, TM * TN>();
      }
    };
    int stage = 0;
    for (int kt = 0; kt + 1 < nk; ++kt) {
      steps_but_last(stage);
      const int next = stage + 1 == ST ? 0 : stage + 1;
      wait_slices<ST - 2, PER>(nk - 2 - kt);
      lds_barrier();
      if (kt + ST < nk) ZK_ISSUE(kt + ST, stage);
      rd(next, 0, 0);
      mma_step(1);
      interleave<TM + TN, TM * TN>();
      stage = next;
    }
    steps_but_last(stage);  // last slice: nothing left to prefetch
    mma_step(1);
  }
#undef ZK_ISSUE
  if constexpr (RES_PREF) {
#pragma unroll
    for (int i = 1; i < NPT; ++i) load_res(i);
    if (!EARLY_GB && p.res_ln) load_gb();
  }
  __syncthreads();  // every wave is done reading the ring; it becomes epilogue space
  form_cols();
  if constexpr (EPI == kEpiQkvAttn) {
    // The tile is the Q, K and V columns of head tn (weights interleaved
    // per head: q, k, v, 64 rows each) for the 256 rows of the sequences
    // the tile holds. They go into LDS as fp16 with their bias, [part][row]
    // [64] with the K/V tile swizzle, and the tile's attention runs from
    // there: Q, K and V never reach HBM.
    static_assert(std::is_same<OP, F16Op>::value && BM == 256 && BN == 192 && MS == 32 &&
                      WM == 4 && WN == 2, "fused QKV attention tile");
    constexpr int HD = 64;
    f16 *qkv = (f16 *)smem;  // 3 x 256 x 64 halves = 96 KB, inside the ring
    const int h32 = lane >> 5;
    // With ln_part the rows of X are the LayerNorm input: Q, K, V are
    // rstd (acc - mean s) + c (see GemmParams), (mean, rstd) per row in LDS.
    float2 *lnt = (float2 *)(smem + 3 * BM * HD * 2);
    static_assert(3 * BM * HD * 2 + BM * 8 <= G::SMEM, "LN table does not fit");
    const bool ln = p.ln_part != nullptr;
    if (ln) {
      if ((int)threadIdx.x < BM) {
        const float2 ms = ln_merge(ln_pr, p.ln_nparts, p.ln_eps);
        lnt[threadIdx.x] = ms;
        if (p.ln_out && tn == 0 && m0 + (int)threadIdx.x < p.M)
          ((float2 *)p.ln_out)[m0 + threadIdx.x] = ms;
      }
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      float2 ms[16];
#pragma unroll
      for (int r = 0; r < 16; ++r)
        ms[r] = ln ? lnt[wm * WTM + i * 32 + 8 * (r >> 2) + 4 * h32 + (r & 3)]
                   : make_float2(0.f, 1.f);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int cb = wn * WTN + j * 32;  // first tile column of the block
        const int d = cb % HD + (lane & 31), n = n0 + cb + (lane & 31);
        const float sv = col_s[j], cv = col_c[j];  // column n's constants
        f16 *dst = qkv + (cb / HD) * (BM * HD);
        // one formula for both cases (no per-element select): without ln,
        // (mean, rstd) = (0, 1) and sv = 0 make it fma(1, fma(-0, 0, acc), c),
        // i.e. acc + c. The outer fma and the fp16 conversion compile to one
        // v_fma_mixlo_f16, which rounds once, to fp16.
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = wm * WTM + i * 32 + 8 * (r >> 2) + 4 * h32 + (r & 3);
          const float v = fmaf(ms[r].y, fmaf(-ms[r].x, sv, acc[i][j][r]), cv);
          dst[row * HD + (((d >> 3) ^ kv_swz(row)) << 3) + (d & 7)] = (f16)v;
        }
      }
    }
    __syncthreads();
    // Wave w owns the 32 queries of tile rows [32 w, 32 w + 32); their
    // sequence's keys are tile rows [sq * seq, +seq).
    const int qr = wave * 32 + (lane & 31);
    const int sq = wave * 32 / p.seq;
    const int b = m0 / p.seq + sq;
    if (b < p.batch) {
      // opaque until here, so that the select below is not formed (and
      // waited for) right after the load at kernel start
      asm volatile("" : "+v"(attn_len));
      int L = p.valid_lens ? attn_len : p.seq;
      L = L < 0 ? 0 : (L > p.seq ? p.seq : L);
      f16x8 qf[HD / 16];
#pragma unroll
      for (int c = 0; c < HD / 16; ++c)
        qf[c] = *(const f16x8 *)(qkv + qr * HD + (((2 * c + h32) ^ kv_swz(qr)) << 3));
      const f16 *Kt = qkv + BM * HD + sq * p.seq * HD, *Vt = Kt + BM * HD;
      f32x16 o[HD / 32];
#pragma unroll
      for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
      float m = -__builtin_inff(), l = 0.f;
      // At most two 64-key tiles (sequences of 64 or 128 tokens), both in
      // LDS: the second tile's Q.K^T is issued before the first tile's
      // softmax, so that its MFMAs can run under that VALU work (the same
      // arithmetic per tile as attn32_tile, in the same order).
      const int ntiles = (L + 63) / 64;
      if (ntiles > 0) {
        // Both tiles are processed whatever the length (a wave-uniform branch
        // would let the compiler hoist the exponentials above it and lose the
        // interleaving): with 64-token sequences tile 1 is tile 0 again, and
        // wherever L <= 64 every key of tile 1 lies at or past L, so its
        // probabilities are 0 and m, l and o stay exactly as they were.
        const int off1 = p.seq > 64 ? 64 * HD : 0;
        f32x16 s0[2], s1[2];
        f16x8 pf0[2][2], pf1[2][2];
        attn32_qk<HD, true, HD>(Kt, qf, lane, s0);
        const float mneg = attn32_softmax_max<HD, false>(s0, 0, L, p.scale_log2, nullptr,
                                                         nullptr, lane, o, m, l);
        // tile 1's 8 K-fragment reads and 8 MFMAs among tile 0's exponentials
        attn32_qk<HD, true, HD>(Kt + off1, qf, lane, s1);
        attn32_softmax_exp<HD>(s0, p.scale_log2, mneg, l, pf0);
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);  // DS reads
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x402, 8, 0);  // VALU incl. exp
        }
        // tile 0's P.V (16 transposing reads, 8 MFMAs) among tile 1's
        // exponentials; tile 1's rescale of o, if any, after it
        float alpha;
        bool resc;
        const float mneg1 = attn32_max_defer(s1, 1, L, p.scale_log2, lane, m, l, alpha, resc);
        attn32_softmax_exp<HD>(s1, p.scale_log2, mneg1, l, pf1);
        attn32_pv<HD, true, HD>(Vt, pf0, lane, o);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS reads
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x402, 8, 0);  // VALU incl. exp
        }
        if (resc) {
#pragma unroll
          for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
        }
        attn32_pv<HD, true, HD>(Vt + off1, pf1, lane, o);
      }
      const int grow = m0 + qr;
      const float inv = l > 0.f ? 1.0f / l : 0.f;
      // (f16)as_f32(o inv) in both layouts: the product rounded to fp32, then
      // to fp16, so that no build fuses it into one rounding in one of them
      if (p.c_pk) {
        // ctx in fragment order (the out-projection's A): the wave's 32 rows
        // are one row block, head tn's 64 columns four 1 KB k-steps. Lane l
        // holds columns 8 g + 4 (l / 32) .. +3 of each 32-column group; one
        // v_permlane32_swap per register pair hands each half of the wave
        // the other half's 4 columns, so that lane l holds columns
        // 8 (l / 32) .. +7 of a k-step (16 bytes, one store per k-step).
        char *F = (char *)p.C + ((int64_t)((m0 + wave * 32) / 32) * (p.ldc / 16) + tn * (HD / 16)) * 1024 +
                  lane * 16;
#pragma unroll
        for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
          for (int kh = 0; kh < 2; ++kh) {
            u32x2 a, b;  // columns 16 kh + 4 (l / 32) and 16 kh + 8 + 4 (l / 32), 4 each
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const f16 a0 = (f16)as_f32(o[dt][8 * kh + 2 * e] * inv);
              const f16 a1 = (f16)as_f32(o[dt][8 * kh + 2 * e + 1] * inv);
              const f16 b0 = (f16)as_f32(o[dt][8 * kh + 4 + 2 * e] * inv);
              const f16 b1 = (f16)as_f32(o[dt][8 * kh + 4 + 2 * e + 1] * inv);
              a[e] = (unsigned)__builtin_bit_cast(unsigned short, a0) |
                     ((unsigned)__builtin_bit_cast(unsigned short, a1) << 16);
              b[e] = (unsigned)__builtin_bit_cast(unsigned short, b0) |
                     ((unsigned)__builtin_bit_cast(unsigned short, b1) << 16);
            }
            // upper lanes' a <-> lower lanes' b: the lower half then holds
            // columns 0-7 of the k-step in (a, b), the upper half 8-15
            u32x4 v;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const auto sw = __builtin_amdgcn_permlane32_swap(a[e], b[e], false, false);
              v[e] = sw[0];
              v[e + 2] = sw[1];
            }
            if (grow < p.M) store_nt((u32x4 *)(F + (dt * 2 + kh) * 1024), v);
          }
      } else if (grow < p.M) {
        f16 *O = (f16 *)p.C + (int64_t)grow * p.ldc + tn * HD;
#pragma unroll
        for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            f16x4 out;
#pragma unroll
            for (int e = 0; e < 4; ++e) out[e] = (f16)as_f32(o[dt][4 * g + e] * inv);
            *(f16x4 *)(O + dt * 32 + 8 * g + 4 * h32) = out;
          }
      }
    }
  } else {
    // Epilogue: per wave, one MS-row stripe at a time.
    constexpr bool RES_STATS = EPI == kEpiResStats;
    constexpr bool LN_IN = EPI == kEpiLnIn || EPI == kEpiLnInGelu;
    constexpr bool RESID = EPI == ZK_EPI_BIAS_RESIDUAL || RES_STATS;
    float *ws = (float *)smem + wave * MS * G::EPITCH;
    // LN_IN: (mean, rstd) of the tile's rows, in LDS beyond the stripes
    float2 *lnt = (float2 *)(smem + G::EPI_BYTES);
    if constexpr (LN_IN) {
      static_assert(G::EPI_BYTES + BM * 8 <= G::SMEM, "LN table does not fit");
      if ((int)threadIdx.x < BM) {
        const float2 ms = ln_merge(ln_pr, p.ln_nparts, p.ln_eps);
        lnt[threadIdx.x] = ms;
        if (p.ln_out && tn == 0 && m0 + (int)threadIdx.x < p.M)
          ((float2 *)p.ln_out)[m0 + threadIdx.x] = ms;
      }
      __syncthreads();
    }
    // int8 output (re-quantisation): bias and residual are fp16; the value is
    // rounded to fp16 first, so the result equals quantising the fp16 output.
    constexpr bool Q8 = std::is_same<OutT, int8_t>::value;
    OutT *C = (OutT *)p.C + (p.splits > 1 ? split * p.split_stride : 0);
    const BiasT *res = (const BiasT *)p.res;
    const float inv_q = Q8 ? 1.0f / p.s_q : 1.0f;
    const bool vec_ok = (p.ldc % 8 == 0) && (Q8 ? aligned8(p.C) : aligned16(p.C)) &&
                        (!RESID || ((p.ldr % 8 == 0) && aligned16(p.res)));
    // this lane's column constants, loaded at kernel start: bias (or LN_IN's
    // offset c) and scale (DEQ's s_x s_w, LN_IN's column sum s)
    const float *bj = col_c, *sj = col_s;
    // the residual's value at (row, col) (RES_STATS with res_ln: its LayerNorm)
    auto resid = [&](int row, int col, float r) {
      if constexpr (RES_STATS) {
        if (p.res_ln) {
          const float2 ms = ((const float2 *)p.res_ln)[row];
          return fmaf((r - ms.x) * ms.y, to_f(((const f16 *)p.res_gamma)[col]),
                      to_f(((const f16 *)p.res_beta)[col]));
        }
      }
      return r;
    };
    constexpr int VPR = WTN / 8;  // 8-column vectors per stripe row
    // fragment-ordered output (p.c_pk): the folded-LayerNorm GELU epilogue of
    // the fp16 32x32 tiles and the re-quantising int8 ones (FFN-up, whose
    // output is FFN-down's A)
    constexpr bool CPK = MS == 32 && ((EPI == kEpiLnInGelu && std::is_same<OutT, f16>::value &&
                                       WTN % 16 == 0) ||
                                      (Q8 && WTN % 32 == 0));
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      // LN_IN: (mean, rstd) of the rows this lane's registers hold
      float2 msr[LN_IN ? R : 1];
      if constexpr (LN_IN) {
#pragma unroll
        for (int r = 0; r < R; ++r)
          msr[r] = lnt[wm * WTM + i * MS + (MS == 32 ? 8 * (r >> 2) + 4 * fch + (r & 3) : 4 * fch + r)];
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int rl = MS == 32 ? 8 * (r >> 2) + 4 * fch + (r & 3) : 4 * fch + r;
          float *dst = ws + rl * G::EPITCH + j * MS + frow;
          if constexpr (std::is_same<OutT, int32_t>::value) {
            *(int *)dst = acc[i][j][r];
          } else if constexpr (LN_IN) {
            // rstd (acc - mean s) + c, then the activation
            const float t = fmaf(msr[r].y, fmaf(-msr[r].x, sj[j], (float)acc[i][j][r]), bj[j]);
            *dst = EPI == kEpiLnInGelu ? gelu_erf_fast(t) : t;
          } else {
            const float v = DEQ ? (float)acc[i][j][r] * sj[j] : (float)acc[i][j][r];
            *dst = epilogue<RES_STATS ? (int)ZK_EPI_BIAS : EPI>(v, bj[j]);
          }
        }
      }
      const int row0 = m0 + wm * WTM + i * MS, col0 = n0 + wn * WTN;
      auto store_vec = [&](int v, int k) {
        const int rl = v / VPR, cl = (v % VPR) * 8;
        const int row = row0 + rl, col = col0 + cl;
        if (row >= p.M || col >= p.N) return;
        float *src = ws + rl * G::EPITCH + cl;
        OutT *dst = C + (int64_t)row * p.ldc + col;
        if (vec_ok && col + 8 <= p.N) {
          const f32x4 lo = *(const f32x4 *)src, hi = *(const f32x4 *)(src + 4);
          if constexpr (std::is_same<OutT, int32_t>::value) {
            *(f32x4 *)dst = lo;  // raw bits of the int32 accumulators
            *(f32x4 *)(dst + 4) = hi;
          } else {
            float o[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            if constexpr (RESID) {
              const BiasT *rp = res + (int64_t)row * p.ldr + col;
              if constexpr (std::is_same<BiasT, f16>::value) {
                const f16x8 rv = RES_PREF ? res_pv[RES_PREF ? i : 0][k] : *(const f16x8 *)rp;
                if (RES_STATS && p.res_ln) {
                  // LN(res): one (mean, rstd) per row, gamma / beta as vectors
                  const float2 ms = RES_PREF ? res_ms[RES_PREF ? i : 0][k]
                                             : ((const float2 *)p.res_ln)[row];
                  const f16x8 g = RES_PREF ? res_g[k] : *(const f16x8 *)((const f16 *)p.res_gamma + col);
                  const f16x8 bb = RES_PREF ? res_b[k] : *(const f16x8 *)((const f16 *)p.res_beta + col);
#pragma unroll
                  for (int e = 0; e < 8; ++e)
                    o[e] += fmaf(((float)rv[e] - ms.x) * ms.y, (float)g[e], (float)bb[e]);
                } else {
#pragma unroll
                  for (int e = 0; e < 8; ++e) o[e] += (float)rv[e];
                }
              } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] += resid(row, col + e, to_f(rp[e]));
              }
            }
            if constexpr (std::is_same<OutT, f16>::value) {
              f16x8 h;
#pragma unroll
              for (int e = 0; e < 8; ++e) h[e] = (f16)o[e];
              store_nt((f16x8 *)dst, h);
              if constexpr (RES_STATS) {  // the stored values, for the statistics
                *(f32x4 *)src = f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
                *(f32x4 *)(src + 4) = f32x4{(float)h[4], (float)h[5], (float)h[6], (float)h[7]};
              }
            } else if constexpr (Q8) {
              float of[8];  // rounded to fp16 first: the fp16 output's quantisation
#pragma unroll
              for (int e = 0; e < 8; ++e) of[e] = (float)(f16)o[e];
              store_nt((u32x2 *)dst, quant8(of, p.s_q, inv_q));
            } else {
              *(f32x4 *)dst = f32x4{o[0], o[1], o[2], o[3]};
              *(f32x4 *)(dst + 4) = f32x4{o[4], o[5], o[6], o[7]};
            }
          }
        } else {
          for (int e = 0; e < 8 && col + e < p.N; ++e) {
            if constexpr (std::is_same<OutT, int32_t>::value) {
              dst[e] = ((const int *)src)[e];
            } else {
              float o = src[e];
              if (RESID) o += resid(row, col + e, to_f(res[(int64_t)row * p.ldr + col + e]));
              if constexpr (Q8) dst[e] = quant1((float)(f16)o, p.s_q, inv_q);
              else dst[e] = (OutT)o;
              if constexpr (RES_STATS) src[e] = (float)(OutT)o;
            }
          }
        }
      };
      if constexpr (CPK) {
        if (p.c_pk) {
          // C in fragment order: the stripe (32 rows, a whole row block) is a
          // run of the consumer's 1 KB A fragments of KC columns (16 fp16 or
          // 32 int8); lane l stores row l % 32, columns KE (l / 32) .. +KE-1
          // of its fragment: 16 bytes
          constexpr int KC = Q8 ? 32 : 16, KE = KC / 2;
          const int rl = lane & 31;
          const int64_t blk = (int64_t)(row0 / 32) * (p.N / KC) + col0 / KC;
#pragma unroll
          for (int kc = 0; kc < WTN / KC; ++kc) {
            const int cl = kc * KC + (lane >> 5) * KE;
            if (row0 + rl < p.M && col0 + cl < p.N) {
              const float *src = ws + rl * G::EPITCH + cl;
              char *dst = (char *)p.C + ((blk + kc) * 64 + lane) * 16;
              if constexpr (Q8) {
                // rounded to fp16 first, as the row-major stores do
                float of[2][8];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                  const f32x4 lo = *(const f32x4 *)(src + 8 * h), hi = *(const f32x4 *)(src + 8 * h + 4);
#pragma unroll
                  for (int e = 0; e < 4; ++e) {
                    of[h][e] = (float)(f16)lo[e];
                    of[h][e + 4] = (float)(f16)hi[e];
                  }
                }
                const u32x2 q0 = quant8(of[0], p.s_q, inv_q), q1 = quant8(of[1], p.s_q, inv_q);
                store_nt((u32x4 *)dst, u32x4{q0[0], q0[1], q1[0], q1[1]});
              } else {
                const f32x4 lo = *(const f32x4 *)src, hi = *(const f32x4 *)(src + 4);
                f16x8 h;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  h[e] = (f16)lo[e];
                  h[e + 4] = (f16)hi[e];
                }
                store_nt((f16x8 *)dst, h);
              }
            }
          }
          continue;
        }
      }
      if constexpr (RES_PREF) {
#pragma unroll
        for (int k = 0; k < NPV; ++k)
          if (lane + 64 * k < MS * VPR) store_vec(lane + 64 * k, k);
      } else {
        for (int v = lane; v < MS * VPR; v += 64) store_vec(v, 0);
      }
      if constexpr (RES_STATS) {
        // (mean, M2) of every kLnSeg-column segment of the stripe's rows,
        // from the stored (rounded) values. Two neighbouring lanes per (row,
        // segment), each over half of it; the halves are merged by Chan's
        // rule: M2 = M2a + M2b + (mean_a - mean_b)^2 * n / 4.
        static_assert(WTN % kLnSeg == 0 && kLnSeg % 8 == 0, "statistics segments");
        constexpr int SEG = WTN / kLnSeg, HALF = kLnSeg / 2;
        for (int v = lane; v < 2 * MS * SEG; v += 64) {  // 2 MS SEG is even: pairs stay together
          const int pr = v >> 1, hf = v & 1;
          const int rl = pr / SEG, sg = pr % SEG;
          const int row = row0 + rl;
          const bool ok = row < p.M && col0 + kLnSeg * sg < p.N;
          float mean = 0.f, m2 = 0.f;
          if (ok) {
            const f32x4 *x4 = (const f32x4 *)(ws + rl * G::EPITCH + kLnSeg * sg + HALF * hf);
            float sum = 0.f;
#pragma unroll
            for (int q = 0; q < HALF / 4; ++q) {
              const f32x4 t = x4[q];
              sum += (t[0] + t[1]) + (t[2] + t[3]);
            }
            mean = sum * (1.0f / HALF);
#pragma unroll
            for (int q = 0; q < HALF / 4; ++q) {
              const f32x4 t = x4[q];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float d = t[e] - mean;
                m2 = fmaf(d, d, m2);
              }
            }
          }
          const float mo = lane_xor1(mean), m2o = lane_xor1(m2);
          if (ok && hf == 0) {
            const float d = mo - mean;
            ((float2 *)p.part_out)[(int64_t)row * (p.N / kLnSeg) + col0 / kLnSeg + sg] =
                make_float2(0.5f * (mean + mo), m2 + m2o + d * d * (0.25f * kLnSeg));
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------ dispatch ----
// Tile configurations (BM, BN, MS, BKB, ST, wave grid); the choice rule is
// in pick_cfg.
//   0: 256x256, 32x32 MFMA, 128-byte slices, 2-stage ring, 8 waves (2 x 4)
//   1: 128x128, 32x32, 128-byte slices, 2-stage ring (2 WG/CU)
//   2: 128x96,  16x16, 128-byte slices, 2-stage ring (2 WG/CU)
//   3: 64x64,   16x16, 128-byte slices, 2-stage ring (up to 5 WG/CU)
//   4: 128x96,  32x32, 128-byte slices, 3-stage ring, 4 waves (4 x 1)
//   5: 256x192, 32x32, 128-byte slices, 2-stage ring, 8 waves (4 x 2)
// The 8-wave tiles put two wavefronts of one workgroup on every SIMD, so
// one wave's barrier or memory wait is covered by the other's MFMAs.
constexpr int kNumCfgs = 6;

// Returns false when no kernel of this configuration implements `epi` for
// these operand types (nothing is launched then): callers turn that into
// ZK_ERR_UNSUPPORTED instead of leaving the output unwritten.
// Sets p's tile counts and XCD grouping for BM x BN tiles; returns the grid.
static int tile_grid(GemmParams &p, int BM, int BN) {
  p.tiles_n = (p.N + BN - 1) / BN;
  p.tiles_m = (p.M + BM - 1) / BM;
  const int grid = p.tiles_m * p.tiles_n * (p.splits > 1 ? p.splits : 1);
  // tile rows per group: enough that one XCD's share of the grid is a
  // rectangle about as tall as it is wide
  int gm = 1;
  const int per_xcd = (grid + 7) / 8;
  while (gm * 2 <= p.tiles_m && gm * gm * 4 <= per_xcd) gm *= 2;
  p.group_m = gm;
  return grid;
}

template <class OP, int BM, int BN, int MS, int BKB, int ST, typename OutT, bool DEQ, int WM = 2,
          int WN = 2>
static bool launch_epi(GemmParams p, int epi, hipStream_t s) {
  const int grid = tile_grid(p, BM, BN);
#define ZK_L(E) \
  (gemm_mfma_kernel<OP, BM, BN, MS, BKB, ST, WM, WN, E, OutT, DEQ><<<grid, 64 * WM * WN, 0, s>>>(p), \
   true)
  switch (epi) {
    case ZK_EPI_NONE: return ZK_L(ZK_EPI_NONE);
    case ZK_EPI_BIAS: return ZK_L(ZK_EPI_BIAS);
    case ZK_EPI_BIAS_GELU_ERF: return ZK_L(ZK_EPI_BIAS_GELU_ERF);
    case ZK_EPI_BIAS_GELU_TANH: return ZK_L(ZK_EPI_BIAS_GELU_TANH);
    case ZK_EPI_BIAS_RESIDUAL:
      if constexpr (!std::is_same<OutT, int8_t>::value) return ZK_L(ZK_EPI_BIAS_RESIDUAL);
      return false;
    case ZK_EPI_BIAS_RELU: return ZK_L(ZK_EPI_BIAS_RELU);
    default:
      // the folded-LayerNorm epilogues: fp16 in and out; statistics need
      // wave tiles of whole kLnSeg-column segments
      if constexpr (std::is_same<OP, F16Op>::value && std::is_same<OutT, f16>::value && !DEQ) {
        if (epi == kEpiLnIn) return ZK_L(kEpiLnIn);
        if (epi == kEpiLnInGelu) return ZK_L(kEpiLnInGelu);
        if constexpr ((BN / WN) % kLnSeg == 0)
          if (epi == kEpiResStats) return ZK_L(kEpiResStats);
      }
      // the residual + statistics epilogue on the dequantised int8 product
      if constexpr (std::is_same<OP, I8Op>::value && std::is_same<OutT, f16>::value && DEQ &&
                    (BN / WN) % kLnSeg == 0)
        if (epi == kEpiResStats) return ZK_L(kEpiResStats);
      return false;
  }
#undef ZK_L
}

// The residual + statistics epilogue on fragment-ordered A (p.a_pk): the
// fp16 128x96 tile of 4 x 1 waves and 3-stage ring that FFN-down runs on
// with row-major A.
template <class OP, bool DEQ, int EPI = kEpiResStats>
static void launch_frag_res_stats(GemmParams p, hipStream_t s) {
  const int grid = tile_grid(p, 128, 96);
  gemm_mfma_kernel<OP, 128, 96, 32, 128, 3, 4, 1, EPI, f16, DEQ, true>
      <<<grid, 256, 0, s>>>(p);
}

// Shape -> configuration, from measurements at the BERT shapes (M = 4096)
// and at square sizes:
//   M >= 1024 and >= 256 tiles of 256x256 (4096^3 and up): the 8-wave
//     256x256 tile;
//   N <= 1024 (out-projection, FFN-down): 64x64 tiles for short K keep every
//     CU busy; for K >= 2048 the 3-stage 128x96 ring (M = 4096, N = 768:
//     256 tiles, one per CU);
//   M >= 1024 and >= 160 tiles of 256x192 (FFN-up: 256, QKV: 192): the
//     8-wave 256x192 tile;
//   otherwise 128x128 once that gives >= 640 tiles, else 128x96.
// Tuning builds only (compiled with -DZK_TUNING): the environment variable
// ZK_GEMM_CFG=<id> forces one configuration for every GEMM and turns split-K
// off. The shipped library has no such switch and always plans by shape.
static int forced_cfg() {
#ifdef ZK_TUNING
  static int forced = -2;
  if (forced == -2) {
    const char *e = getenv("ZK_GEMM_CFG");
    forced = e ? atoi(e) : -1;
  }
  return forced >= 0 && forced < kNumCfgs ? forced : -1;
#else
  return -1;
#endif
}

static int pick_cfg(int M, int N, int K) {
  if (forced_cfg() >= 0) return forced_cfg();
  const int64_t tm256 = (M + 255) / 256;
  const int64_t t256 = tm256 * ((N + 255) / 256);
  if (M >= 1024 && N > 1024 && t256 >= 256) {
    // 256x256, unless 256x192 tiles take fewer whole rounds of 256 CUs times
    // their area (units of 256x64): QKV at s512 (M = 16384, N = 2304) is 576
    // tiles of 256x256, three rounds with the last a quarter full, or 768
    // tiles of 256x192, three full rounds of smaller tiles
    const int64_t t192n = tm256 * ((N + 191) / 192);
    const int64_t c256 = (t256 + 255) / 256 * 4, c192 = (t192n + 255) / 256 * 3;
    return c192 < c256 ? 5 : 0;
  }
  // 256x192 tiles whenever they fill at least one wave of 256 CUs, also for
  // N <= 1024 at large M (s512: M = 16384, N = 768 gives exactly 256 tiles;
  // FFN-down 96.5 -> 73.6 us, out-projection 33.6 -> 24.2 us against the
  // small tiles below)
  const int64_t t192 = tm256 * ((N + 191) / 192);
  if (M >= 1024 && t192 >= 256) return 5;
  // the 3-stage 128x96 ring for deep K (FFN-down, K = 3072, fp16 and int8),
  // 64x64 otherwise. At M = 4096, N = 768 the 128x96 tile gives 256 tiles
  // (one per CU) where 128x128 left 64 CUs idle: the fp16 encoder is 1.8-2.8%
  // and the INT8-FFN encoder 0.5-1.5% faster per step (one-process A/Bs in
  // both orders, identical output). Timed alone, the int8 FFN-down is
  // faster on 64x64 than on the 128x128 ring (16.3 against 18.0 us), but
  // inside the encoder the ring won (1.212 against 1.234 ms per step), so
  // encoder figures decide.
  // Below 1024 rows (a few sequences: the per-GPU share of a data-parallel
  // batch, or serving) the 64x64 tile whenever the larger ones would leave
  // CUs idle: at M = 512 (four 128-token sequences) the QKV projection is 96
  // tiles of 128x96 or 288 of 64x64, FFN-down 32 tiles of 128x96 or 96 of
  // 64x64 (which split-K then doubles when a workspace is given).
  const int64_t t96 = (int64_t)((M + 127) / 128) * ((N + 95) / 96);
  if (M < 1024 && t96 < 256) return 3;
  if (N <= 1024) return K >= 2048 ? 4 : 3;
  if (M >= 1024 && t192 >= 160) return 5;
  const int64_t t128 = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
  return t128 >= 640 ? 1 : 2;
}

// Returns whether a kernel was launched (see launch_epi).
template <class OP, typename OutT, bool DEQ>
[[nodiscard]] static bool launch_mfma(GemmParams p, int epi, hipStream_t s, int cfg = -1) {
  switch (cfg >= 0 ? cfg : pick_cfg(p.M, p.N, p.K)) {
    case 0: return launch_epi<OP, 256, 256, 32, 128, 2, OutT, DEQ, 2, 4>(p, epi, s);
    case 1: return launch_epi<OP, 128, 128, 32, 128, 2, OutT, DEQ>(p, epi, s);
    case 2: return launch_epi<OP, 128, 96, 16, 128, 2, OutT, DEQ>(p, epi, s);
    case 4: return launch_epi<OP, 128, 96, 32, 128, 3, OutT, DEQ, 4, 1>(p, epi, s);
    case 5: return launch_epi<OP, 256, 192, 32, 128, 2, OutT, DEQ, 4, 2>(p, epi, s);
    default: return launch_epi<OP, 64, 64, 16, 128, 2, OutT, DEQ>(p, epi, s);
  }
}

// The status of a GEMM entry point after launch_mfma: unsupported when no
// kernel implements the epilogue for the chosen tile, else the launch check.
static int launched(bool ok, const char *who, int epi) {
  if (!ok) return fail(ZK_ERR_UNSUPPORTED, "%s: epilogue %d has no kernel for this shape", who, epi);
  return check_launch(who);
}

// --------------------------------------------------------------- split-K --
// Problems whose 64x64 tiles cannot fill the GPU (small M, e.g. one
// sequence of 128 tokens) are split along K: workgroup (tile, split) runs
// the 64x64 kernel over its K range and writes the raw fp32 partial tile to
// a caller-provided workspace; splitk_reduce then sums the partials in split
// order (deterministic) and applies the epilogue. Only products of fewer than
// 128 tiles split, into at most 512 / t64 splits, so the partials (splits x
// M x N fp32) never exceed 512 x 64 x 64 x 4 bytes = 8 MiB.
struct SplitPlan {
  int splits;  // 1: no split
  int nk_per;  // 128-byte K slices per split
};

static SplitPlan plan_split(int64_t M, int64_t N, int64_t K, int elem) {
  SplitPlan sp{1, 0};
  if (forced_cfg() >= 0) return sp;
  const int64_t t64 = ((M + 63) / 64) * ((N + 63) / 64);
  const int64_t nk_all = (K * elem + 127) / 128;
  if (t64 >= 128 || nk_all < 4) return sp;
  int64_t splits = 256 / t64;
  if (splits > 16) splits = 16;
  if (splits > nk_all / 2) splits = nk_all / 2;
  // Deep K (>= 24 slices): up to two workgroups per CU, keeping at least 12
  // slices per split. At M = 512 (four 128-token sequences) FFN-down
  // (K = 3072) then runs 4 splits instead of 2: the b4 s128 encoder 0.752
  // -> 0.677 ms per step, b1 and b2 unchanged (their plan is the same).
  // Letting shallow products (QKV, out-projection, FFN-up) follow the same
  // rule left them unsplit: b1 0.605 -> 0.628 ms.
  if (nk_all >= 24) {
    int64_t deep = 512 / t64;
    if (deep > 16) deep = 16;
    if (deep > nk_all / 12) deep = nk_all / 12;
    if (deep > splits) splits = deep;
  }
  if (splits < 2) return sp;
  const int64_t per = (nk_all + splits - 1) / splits;
  splits = (nk_all + per - 1) / per;  // no empty split
  if (splits < 2) return sp;
  return SplitPlan{(int)splits, (int)per};
}

static int64_t split_ws_bytes(int64_t M, int64_t N, const SplitPlan &sp) {
  return sp.splits > 1 ? (int64_t)sp.splits * M * N * (int64_t)sizeof(float) : 0;
}

template <int EPI, typename OutT>
__global__ __launch_bounds__(256) void splitk_reduce(const float *__restrict__ ws, int splits,
                                                     int64_t stride, int M, int N,
                                                     const OutT *__restrict__ bias,
                                                     const OutT *__restrict__ res, int64_t ldr,
                                                     OutT *__restrict__ C, int64_t ldc) {
  const int64_t total = (int64_t)M * N;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += step) {
    const int64_t m = i / N, n = i % N;
    float v = sum_splits<float>(ws + i, splits, stride);
    v = epilogue<EPI>(v, EPI != ZK_EPI_NONE ? to_f(bias[n]) : 0.f);
    if (EPI == ZK_EPI_BIAS_RESIDUAL) v += to_f(res[m * ldr + n]);
    C[m * ldc + n] = (OutT)as_f32(v);  // rounded to fp32, then to OutT, as the GEMM epilogue
  }
}

// splitk_reduce on four consecutive columns per thread: 16-byte partial
// loads and one 8- or 16-byte store (N, ldc and ldr multiples of 4, aligned
// operands). The same sum in the same order as splitk_reduce.
template <int EPI, typename OutT>
__global__ __launch_bounds__(256) void splitk_reduce4(const float *__restrict__ ws, int splits,
                                                      int64_t stride, int M, int N,
                                                      const OutT *__restrict__ bias,
                                                      const OutT *__restrict__ res, int64_t ldr,
                                                      OutT *__restrict__ C, int64_t ldc) {
  typedef OutT OutT4 __attribute__((ext_vector_type(4)));
  const int64_t total = (int64_t)M * N / 4;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += step) {
    const int64_t e = 4 * i, m = e / N, n = e % N;
    f32x4 v = sum_splits<f32x4>(ws + e, splits, stride);
    OutT4 b4 = {}, r4 = {}, o4;
    if (EPI != ZK_EPI_NONE) b4 = *(const OutT4 *)(bias + n);
    if (EPI == ZK_EPI_BIAS_RESIDUAL) r4 = *(const OutT4 *)(res + m * ldr + n);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float t = epilogue<EPI>(v[k], EPI != ZK_EPI_NONE ? to_f(b4[k]) : 0.f);
      if (EPI == ZK_EPI_BIAS_RESIDUAL) t += to_f(r4[k]);
      o4[k] = (OutT)as_f32(t);
    }
    *(OutT4 *)(C + m * ldc + n) = o4;
  }
}

// p describes the final product (C, ldc, bias, residual); the partials go to
// ws (at least split_ws_bytes). OP is F16Op or F32Op.
// Returns whether both kernels were launched (false for an epilogue the
// reduction does not implement; nothing is launched then).
template <class OP, typename OutT>
[[nodiscard]] static bool launch_split(GemmParams p, int epi, const SplitPlan &sp, float *ws,
                                       hipStream_t s) {
  switch (epi) {
    case ZK_EPI_NONE: case ZK_EPI_BIAS: case ZK_EPI_BIAS_GELU_ERF: case ZK_EPI_BIAS_GELU_TANH:
    case ZK_EPI_BIAS_RESIDUAL: case ZK_EPI_BIAS_RELU: break;
    default: return false;
  }
  GemmParams q = p;
  q.C = ws;
  q.ldc = p.N;
  q.bias = nullptr;
  q.res = nullptr;
  q.splits = sp.splits;
  q.nk_per = sp.nk_per;
  q.split_stride = (int64_t)p.M * p.N;
  if (!launch_mfma<OP, float, false>(q, ZK_EPI_NONE, s, 3)) return false;
  const OutT *bias = (const OutT *)p.bias, *res = (const OutT *)p.res;
  OutT *C = (OutT *)p.C;
  // four columns per thread when every row starts on a 4-element boundary
  constexpr int64_t VB = 4 * sizeof(OutT);  // bytes of four outputs
  const bool vec = p.N % 4 == 0 && p.ldc % 4 == 0 && aligned16(ws) && (uintptr_t)C % VB == 0 &&
                   (!bias || (uintptr_t)bias % VB == 0) &&
                   (epi != ZK_EPI_BIAS_RESIDUAL || (p.ldr % 4 == 0 && (uintptr_t)res % VB == 0));
  const int64_t total = (int64_t)p.M * p.N / (vec ? 4 : 1);
  int64_t g = (total + 255) / 256;
  if (g > 4096) g = 4096;
#define ZK_R(E)                                                                              \
  do {                                                                                       \
    if (vec)                                                                                 \
      splitk_reduce4<E, OutT><<<(unsigned)g, 256, 0, s>>>(ws, sp.splits, q.split_stride,   \
                                                          p.M, p.N, bias, res, p.ldr, C,   \
                                                          p.ldc);                          \
    else                                                                                     \
      splitk_reduce<E, OutT><<<(unsigned)g, 256, 0, s>>>(ws, sp.splits, q.split_stride,    \
                                                         p.M, p.N, bias, res, p.ldr, C,    \
                                                         p.ldc);                           \
  } while (0)
  switch (epi) {
    case ZK_EPI_NONE: ZK_R(ZK_EPI_NONE); break;
    case ZK_EPI_BIAS: ZK_R(ZK_EPI_BIAS); break;
    case ZK_EPI_BIAS_GELU_ERF: ZK_R(ZK_EPI_BIAS_GELU_ERF); break;
    case ZK_EPI_BIAS_GELU_TANH: ZK_R(ZK_EPI_BIAS_GELU_TANH); break;
    case ZK_EPI_BIAS_RESIDUAL: ZK_R(ZK_EPI_BIAS_RESIDUAL); break;
    case ZK_EPI_BIAS_RELU: ZK_R(ZK_EPI_BIAS_RELU); break;
  }
#undef ZK_R
  return true;
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

// The MFMA kernel addresses a tile's rows through a buffer descriptor of
// (rows - 1) * ld + K bytes (rows <= 256) with 32-bit offsets, and pushes
// K-tail chunks out of range with the offset 0x7ffffff0; both operands'
// spans must stay below it.
static int check_span(const char *who, int64_t lda, int64_t ldb, int64_t K, int elem) {
  const int64_t lim = 0x7ffffff0LL;
  if (255 * lda * elem + K * elem >= lim || 255 * ldb * elem + K * elem >= lim)
    return fail(ZK_ERR_UNSUPPORTED,
                "%s: leading dimension / K too large for 32-bit tile addressing", who);
  return ZK_OK;
}

}  // namespace zk

using namespace zk;

int zk::gemm_f16_impl(const void *A, const void *B, void *C, int64_t M, int64_t N, int64_t K,
                      int64_t lda, int64_t ldb, int64_t ldc, int trans_b, int out_dtype,
                      const void *bias, const void *residual, int64_t ldr, int epilogue,
                      void *ws, int64_t ws_bytes, void *stream) {
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
  if ((st = check_span("zk_gemm_f16", lda, ldb, K, 2))) return st;
  GemmParams p{A, B, C, (int)M, (int)N, (int)K, lda, ldb, ldc, bias, residual, ldr, 1.f, nullptr, 0};
  hipStream_t s = as_stream(stream);
  const SplitPlan sp = plan_split(M, N, K, 2);
  bool ok;
  if (ws && sp.splits > 1 && ws_bytes >= split_ws_bytes(M, N, sp) && aligned16(ws)) {
    if (out_dtype == ZK_F16) ok = launch_split<F16Op, f16>(p, epilogue, sp, (float *)ws, s);
    else ok = launch_split<F16Op, float>(p, epilogue, sp, (float *)ws, s);
  } else if (out_dtype == ZK_F16) {
    ok = launch_mfma<F16Op, f16, false>(p, epilogue, s);
  } else {
    ok = launch_mfma<F16Op, float, false>(p, epilogue, s);
  }
  return launched(ok, "zk_gemm_f16", epilogue);
}

extern "C" int zk_gemm_f16(const void *A, const void *B, void *C, int64_t M,
                           int64_t N, int64_t K, int64_t lda, int64_t ldb,
                           int64_t ldc, int trans_b, int out_dtype,
                           const void *bias, const void *residual, int64_t ldr,
                           int epilogue, void *stream) {
  return gemm_f16_impl(A, B, C, M, N, K, lda, ldb, ldc, trans_b, out_dtype, bias, residual, ldr,
                       epilogue, nullptr, 0, stream);
}

extern "C" int zk_gemm_f16_ws(const void *A, const void *B, void *C, int64_t M, int64_t N,
                              int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int trans_b,
                              int out_dtype, const void *bias, const void *residual,
                              int64_t ldr, int epilogue, void *workspace, int64_t ws_bytes,
                              void *stream) {
  if (ws_bytes < 0) return fail(ZK_ERR_INVALID, "zk_gemm_f16_ws: negative workspace size");
  return gemm_f16_impl(A, B, C, M, N, K, lda, ldb, ldc, trans_b, out_dtype, bias, residual, ldr,
                       epilogue, workspace, ws_bytes, stream);
}

// Linear + residual + LayerNorm. A product that splits along K (and whose
// rows the wave LayerNorm can hold) runs as its split partials plus one
// LayerNorm launch that forms the rows from the partials; anything else as
// zk_gemm_f16_ws into T followed by zk_layernorm. Both give the pair's
// result bit for bit. Below 2048 rows of at most 1024 values each row gets a
// workgroup of four wavefronts to form it (BERT encoder per step, s128,
// pair -> partials: b1 0.602 -> 0.555 ms, b2 0.635 -> 0.581, b4 0.679 ->
// 0.626); otherwise one wavefront per row reads every split of its row,
// which needs at least 32 rows per split to pay (with it b1, 6 and 10
// splits of 128 rows, measured 0.604 -> 0.621 ms, b2 0.617, b4 0.646).
extern "C" int zk_gemm_f16_add_ln(const void *A, const void *W, const void *bias, const void *R,
                                  const void *gamma, const void *beta, void *T, void *Y,
                                  int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw,
                                  float eps, void *workspace, int64_t ws_bytes, void *stream) {
  const char *who = "zk_gemm_f16_add_ln";
  int st = check_dims(who, M, N, K);
  if (st) return st;
  if (M == 0 || N == 0) return ZK_OK;
  if (!A || !W || !bias || !R || !gamma || !beta || !T || !Y)
    return fail(ZK_ERR_INVALID, "%s: null pointer", who);
  if (!(eps >= 0.0f)) return fail(ZK_ERR_INVALID, "%s: eps must be >= 0", who);
  if (ws_bytes < 0) return fail(ZK_ERR_INVALID, "%s: negative workspace size", who);
  if (lda < K || ldw < K) return fail(ZK_ERR_INVALID, "%s: leading dimension too small", who);
  if (K == 0) return fail(ZK_ERR_UNSUPPORTED, "%s: K == 0", who);
  if (K % 8 || lda % 8 || ldw % 8 || !aligned16(A) || !aligned16(W))
    return fail(ZK_ERR_UNSUPPORTED,
                "%s: K, lda, ldw must be multiples of 8 and A, W 16-byte aligned", who);
  if ((st = check_span(who, lda, ldw, K, 2))) return st;
  hipStream_t s = as_stream(stream);
  const SplitPlan sp = plan_split(M, N, K, 2);
  const float *ws = (const float *)workspace;
  const bool wide = ln_partials_wide_ok(M, N), narrow = !wide && sp.splits * 32 <= M;
  if (ws && sp.splits > 1 && ws_bytes >= split_ws_bytes(M, N, sp) && (narrow || wide) &&
      ln_partials_ok(ws, M * N, bias, R, gamma, beta, Y, M, N)) {
    GemmParams q{A, W, workspace, (int)M, (int)N, (int)K, lda, ldw, N, nullptr, nullptr, 0, 1.f,
                 nullptr, 0};
    q.splits = sp.splits;
    q.nk_per = sp.nk_per;
    q.split_stride = M * N;
    if (!launch_mfma<F16Op, float, false>(q, ZK_EPI_NONE, s, 3))
      return fail(ZK_ERR_UNSUPPORTED, "%s: no partial-product kernel for this shape", who);
    if ((st = check_launch(who))) return st;
    return ln_add_partials_f16(ws, sp.splits, M * N, bias, R, gamma, beta, Y, M, N, eps, wide, s);
  }
  st = gemm_f16_impl(A, W, T, M, N, K, lda, ldw, N, 1, ZK_F16, bias, nullptr, 0, ZK_EPI_BIAS,
                     workspace, ws_bytes, stream);
  if (st) return st;
  return zk_layernorm(T, R, gamma, beta, Y, M, N, eps, ZK_F16, stream);
}

// Fused QKV projection + attention (sequences of 64 or 128 tokens, head dim
// 64): one 256 x 192 tile per workgroup, the q, k and v columns of one head
// for 256 rows, with the attention of the tile's sequences in its epilogue.
static void launch_qkv_attn(GemmParams p, hipStream_t s) {
  p.tiles_n = p.N / 192;
  p.tiles_m = (p.M + 255) / 256;
  const int grid = p.tiles_m * p.tiles_n;
  int gm = 1;
  const int per_xcd = (grid + 7) / 8;
  while (gm * 2 <= p.tiles_m && gm * gm * 4 <= per_xcd) gm *= 2;
  p.group_m = gm;
  gemm_mfma_kernel<F16Op, 256, 192, 32, 128, 2, 4, 2, kEpiQkvAttn, f16, false>
      <<<grid, 512, 0, s>>>(p);
}

static int qkv_attn_impl(const char *who, const void *X, const void *Wqkv, const void *bqkv,
                         const float *ln_part, float ln_eps, const float *ln_s,
                         const float *ln_c, float *ln_out, void *ctx, int64_t batch,
                         int64_t seq, int64_t hidden, int64_t heads, const int32_t *valid_lens,
                         float scale, void *stream, bool frag = false) {
  if (batch < 0 || seq <= 0 || hidden <= 0 || heads <= 0)
    return fail(ZK_ERR_INVALID, "%s: bad size", who);
  if (batch == 0) return ZK_OK;
  if (!X || !Wqkv || !ctx) return fail(ZK_ERR_INVALID, "%s: null pointer", who);
  if (!ln_part && !bqkv) return fail(ZK_ERR_INVALID, "%s: null bias", who);
  if (ln_part && (!ln_s || !ln_c || !(ln_eps >= 0.f)))
    return fail(ZK_ERR_INVALID, "%s: LayerNorm needs column sums, offsets and eps >= 0", who);
  if (!aligned8(ln_part) || !aligned8(ln_out))
    return fail(ZK_ERR_UNSUPPORTED, "%s: statistics arrays must be 8-byte aligned", who);
  if (ln_part && (hidden % kLnSeg || hidden / kLnSeg > kLnMaxParts))
    return fail(ZK_ERR_UNSUPPORTED, "%s: hidden must be a multiple of %d, at most %d", who,
                kLnSeg, kLnSeg * kLnMaxParts);
  if (hidden != heads * 64)
    return fail(ZK_ERR_UNSUPPORTED, "%s: head dim must be 64 (hidden %lld, heads %lld)", who,
                (long long)hidden, (long long)heads);
  if (seq != 64 && seq != 128)
    return fail(ZK_ERR_UNSUPPORTED, "%s: seq must be 64 or 128 (got %lld)", who, (long long)seq);
  if (!(scale > 0.0f) || scale == __builtin_inff())
    return fail(ZK_ERR_INVALID, "%s: scale must be finite and > 0", who);
  if (batch > 0x7fffffff / seq) return fail(ZK_ERR_UNSUPPORTED, "%s: batch * seq exceeds int32", who);
  const int64_t M = batch * seq, N = 3 * hidden, K = hidden;
  int st = check_dims(who, M, N, K);
  if (st) return st;
  if (!aligned16(X) || !aligned16(Wqkv) || !aligned8(ctx))
    return fail(ZK_ERR_UNSUPPORTED, "%s: X and Wqkv must be 16-byte, ctx 8-byte aligned", who);
  if (frag && !aligned16(ctx))
    return fail(ZK_ERR_UNSUPPORTED, "%s: ctx in fragment order must be 16-byte aligned", who);
  if ((st = check_span(who, K, K, K, 2))) return st;
  GemmParams p{X, Wqkv, ctx, (int)M, (int)N, (int)K, K, K, hidden, bqkv, nullptr, 0, 1.f, nullptr, 0};
  p.seq = (int)seq;
  p.batch = (int)batch;
  p.valid_lens = valid_lens;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.ln_part = ln_part;
  p.ln_nparts = (int)(K / kLnSeg);
  p.ln_eps = ln_eps;
  p.ln_s = ln_s;
  p.ln_c = ln_c;
  p.ln_out = ln_out;
  p.c_pk = frag;
  launch_qkv_attn(p, as_stream(stream));
  return check_launch(who);
}

extern "C" int zk_qkv_attn_f16(const void *X, const void *Wqkv, const void *bqkv, void *ctx,
                               int64_t batch, int64_t seq, int64_t hidden, int64_t heads,
                               const int32_t *valid_lens, float scale, void *stream) {
  return qkv_attn_impl("zk_qkv_attn_f16", X, Wqkv, bqkv, nullptr, 0.f, nullptr, nullptr, nullptr,
                       ctx, batch, seq, hidden, heads, valid_lens, scale, stream);
}

extern "C" int zk_qkv_attn_f16_ln(const void *X, const void *Wqkv, const float *ln_part,
                                  float ln_eps, const float *ln_s, const float *ln_c,
                                  float *ln_out, void *ctx, int64_t batch, int64_t seq,
                                  int64_t hidden, int64_t heads, const int32_t *valid_lens,
                                  float scale, void *stream) {
  if (!ln_part) return fail(ZK_ERR_INVALID, "zk_qkv_attn_f16_ln: null statistics");
  return qkv_attn_impl("zk_qkv_attn_f16_ln", X, Wqkv, nullptr, ln_part, ln_eps, ln_s, ln_c,
                       ln_out, ctx, batch, seq, hidden, heads, valid_lens, scale, stream);
}

extern "C" int zk_qkv_attn_f16_frag(const void *X, const void *Wqkv, const void *bqkv,
                                    const float *ln_part, float ln_eps, const float *ln_s,
                                    const float *ln_c, float *ln_out, void *ctx, int64_t batch,
                                    int64_t seq, int64_t hidden, int64_t heads,
                                    const int32_t *valid_lens, float scale, void *stream) {
  return qkv_attn_impl("zk_qkv_attn_f16_frag", X, Wqkv, ln_part ? nullptr : bqkv, ln_part,
                       ln_eps, ln_s, ln_c, ln_out, ctx, batch, seq, hidden, heads, valid_lens,
                       scale, stream, true);
}

// Operand checks of the folded-LayerNorm GEMMs: fp16, W[N,K], dense-enough
// rows in multiples of 8, 16-byte aligned.
static int check_ln_gemm(const char *who, const void *A, const void *W, const void *C, int64_t M,
                         int64_t N, int64_t K, int64_t lda, int64_t ldw, int64_t ldc) {
  int st = check_dims(who, M, N, K);
  if (st) return st;
  if (!A || !W || !C) return fail(ZK_ERR_INVALID, "%s: null pointer", who);
  if (lda < K || ldw < K || ldc < N) return fail(ZK_ERR_INVALID, "%s: leading dimension too small", who);
  if (K == 0 || K % 8 || lda % 8 || ldw % 8 || ldc % 8 || !aligned16(A) || !aligned16(W) ||
      !aligned16(C))
    return fail(ZK_ERR_UNSUPPORTED,
                "%s: K and the leading dimensions must be multiples of 8, operands 16-byte "
                "aligned", who);
  return check_span(who, lda, ldw, K, 2);
}

static int check_i8(const char *who, const int8_t *A, const int8_t *W, const void *C, int64_t M,
                    int64_t N, int64_t K, int64_t lda, int64_t ldw, int64_t ldc, int epilogue);

// The residual / statistics operands of zk_gemm_f16_res_stats and
// zk_gemm_i8_res_stats, checked, then the launch on the configurations whose
// wave tiles are one statistics segment wide: 256x192 (8 waves) once it
// fills the CUs, else 128x96 (4 waves).
template <class OP, bool DEQ>
static int res_stats_run(const char *who, GemmParams p, const float *res_ln, const void *res_gamma,
                         const void *res_beta, float *part_out, void *stream) {
  const int64_t M = p.M, N = p.N;
  if (!p.bias || !p.res || !part_out)
    return fail(ZK_ERR_INVALID, "%s: null bias, residual or statistics", who);
  if (N % kLnSeg) return fail(ZK_ERR_UNSUPPORTED, "%s: N must be a multiple of %d", who, kLnSeg);
  if (res_ln && (!res_gamma || !res_beta))
    return fail(ZK_ERR_INVALID, "%s: residual LayerNorm needs gamma and beta", who);
  if (p.ldr < N) return fail(ZK_ERR_INVALID, "%s: ldr < N", who);
  if (p.ldr % 8 || !aligned16(p.res))
    return fail(ZK_ERR_UNSUPPORTED, "%s: residual rows must be 16-byte aligned", who);
  if (!aligned8(res_ln) || !aligned8(part_out) || !aligned16(res_gamma) || !aligned16(res_beta))
    return fail(ZK_ERR_UNSUPPORTED,
                "%s: statistics 8-byte, gamma and beta 16-byte aligned", who);
  p.res_ln = res_ln;
  p.res_gamma = res_gamma;
  p.res_beta = res_beta;
  p.part_out = part_out;
  if (p.a_pk) {
    launch_frag_res_stats<OP, DEQ>(p, as_stream(stream));
    return launched(true, who, kEpiResStats);
  }
  const int64_t t192 = (M + 255) / 256 * (N / 192);
  const bool ok = launch_mfma<OP, f16, DEQ>(p, kEpiResStats, as_stream(stream),
                                            M >= 1024 && N % 192 == 0 && t192 >= 160 ? 5 : 4);
  return launched(ok, who, kEpiResStats);
}

extern "C" int zk_gemm_f16_res_stats(const void *A, const void *W, void *C, int64_t M, int64_t N,
                                     int64_t K, int64_t lda, int64_t ldw, int64_t ldc,
                                     const void *bias, const void *res, int64_t ldr,
                                     const float *res_ln, const void *res_gamma,
                                     const void *res_beta, float *part_out, void *stream) {
  const char *who = "zk_gemm_f16_res_stats";
  int st = check_ln_gemm(who, A, W, C, M, N, K, lda, ldw, ldc);
  if (st) return st;
  if (M == 0 || N == 0) return ZK_OK;
  GemmParams p{A, W, C, (int)M, (int)N, (int)K, lda, ldw, ldc, bias, res, ldr, 1.f, nullptr, 0};
  return res_stats_run<F16Op, false>(who, p, res_ln, res_gamma, res_beta, part_out, stream);
}

extern "C" int zk_gemm_f16_frag(const void *A, const void *W, void *C, int64_t M, int64_t N,
                                int64_t K, int64_t ldw, int64_t ldc, const void *bias,
                                void *stream) {
  const char *who = "zk_gemm_f16_frag";
  int st = check_ln_gemm(who, A, W, C, M, N, K, K, ldw, ldc);
  if (st) return st;
  if (M == 0 || N == 0) return ZK_OK;
  if (K % 64) return fail(ZK_ERR_UNSUPPORTED, "%s: K must be a multiple of 64", who);
  if (!bias) return fail(ZK_ERR_INVALID, "%s: null bias", who);
  GemmParams p{A, W, C, (int)M, (int)N, (int)K, K, ldw, ldc, bias, nullptr, 0, 1.f, nullptr, 0};
  p.a_pk = A;
  launch_frag_res_stats<F16Op, false, ZK_EPI_BIAS>(p, as_stream(stream));
  return check_launch(who);
}

extern "C" int zk_gemm_f16_res_stats_frag(const void *A, const void *W, void *C, int64_t M,
                                          int64_t N, int64_t K, int64_t ldw, int64_t ldc,
                                          const void *bias, const void *res, int64_t ldr,
                                          const float *res_ln, const void *res_gamma,
                                          const void *res_beta, float *part_out, void *stream) {
  const char *who = "zk_gemm_f16_res_stats_frag";
  int st = check_ln_gemm(who, A, W, C, M, N, K, K, ldw, ldc);
  if (st) return st;
  if (M == 0 || N == 0) return ZK_OK;
  if (K % 64) return fail(ZK_ERR_UNSUPPORTED, "%s: K must be a multiple of 64", who);
  GemmParams p{A, W, C, (int)M, (int)N, (int)K, K, ldw, ldc, bias, res, ldr, 1.f, nullptr, 0};
  p.a_pk = A;
  return res_stats_run<F16Op, false>(who, p, res_ln, res_gamma, res_beta, part_out, stream);
}

extern "C" int zk_gemm_i8_res_stats(const int8_t *A, const int8_t *W, void *C, int64_t M,
                                    int64_t N, int64_t K, int64_t lda, int64_t ldw, int64_t ldc,
                                    float s_x, const float *s_w, const void *bias,
                                    const void *res, int64_t ldr, const float *res_ln,
                                    const void *res_gamma, const void *res_beta, float *part_out,
                                    void *stream) {
  const char *who = "zk_gemm_i8_res_stats";
  int st = check_i8(who, A, W, C, M, N, K, lda, ldw, ldc, ZK_EPI_BIAS);
  if (st || M == 0 || N == 0) return st;
  if (!s_w || !(s_x > 0.f)) return fail(ZK_ERR_INVALID, "%s: s_w and s_x > 0 are required", who);
  if (ldc % 8 || !aligned16(C))
    return fail(ZK_ERR_UNSUPPORTED, "%s: ldc must be a multiple of 8 and C 16-byte aligned", who);
  GemmParams p{A, W, C, (int)M, (int)N, (int)K, lda, ldw, ldc, bias, res, ldr, s_x, s_w, 0};
  return res_stats_run<I8Op, true>(who, p, res_ln, res_gamma, res_beta, part_out, stream);
}

static int gemm_f16_ln(const char *who, const void *A, const void *W, void *C, int64_t M,
                       int64_t N, int64_t K, int64_t lda, int64_t ldw, int64_t ldc,
                       const float *ln_part, float ln_eps, const float *ln_s, const float *ln_c,
                       float *ln_out, int epilogue, bool frag, void *stream) {
  int st = check_ln_gemm(who, A, W, C, M, N, K, lda, ldw, ldc);
  if (st) return st;
  if (M == 0 || N == 0) return ZK_OK;
  if (!ln_part || !ln_s || !ln_c || !(ln_eps >= 0.f))
    return fail(ZK_ERR_INVALID, "%s: null statistics, column sums or offsets, or eps < 0", who);
  if (epilogue != ZK_EPI_BIAS && epilogue != ZK_EPI_BIAS_GELU_ERF)
    return fail(ZK_ERR_UNSUPPORTED, "%s: epilogue must be ZK_EPI_BIAS or ZK_EPI_BIAS_GELU_ERF", who);
  if (K % kLnSeg || K / kLnSeg > kLnMaxParts)
    return fail(ZK_ERR_UNSUPPORTED, "%s: K must be a multiple of %d, at most %d", who, kLnSeg,
                kLnSeg * kLnMaxParts);
  if (!aligned8(ln_part) || !aligned8(ln_out) || !aligned16(ln_s) || !aligned16(ln_c))
    return fail(ZK_ERR_UNSUPPORTED,
                "%s: statistics 8-byte, column sums and offsets 16-byte aligned", who);
  GemmParams p{A, W, C, (int)M, (int)N, (int)K, lda, ldw, ldc, nullptr, nullptr, 0, 1.f, nullptr, 0};
  p.ln_part = ln_part;
  p.ln_nparts = (int)(K / kLnSeg);
  p.ln_eps = ln_eps;
  p.ln_s = ln_s;
  p.ln_c = ln_c;
  p.ln_out = ln_out;
  const int epi = epilogue == ZK_EPI_BIAS ? kEpiLnIn : kEpiLnInGelu;
  int cfg = pick_cfg(p.M, p.N, p.K);
  if (frag) {
    // every 32x32-MFMA tile (0, 1, 4, 5) has the fragment-ordered store; the
    // 16x16 ones (2, 3) give way to the 128x96 tile
    p.c_pk = 1;
    if (cfg == 2 || cfg == 3) cfg = 4;
  }
  return launched(launch_mfma<F16Op, f16, false>(p, epi, as_stream(stream), cfg), who, epi);
}

extern "C" int zk_gemm_f16_ln(const void *A, const void *W, void *C, int64_t M, int64_t N,
                              int64_t K, int64_t lda, int64_t ldw, int64_t ldc,
                              const float *ln_part, float ln_eps, const float *ln_s,
                              const float *ln_c, float *ln_out, int epilogue, void *stream) {
  return gemm_f16_ln("zk_gemm_f16_ln", A, W, C, M, N, K, lda, ldw, ldc, ln_part, ln_eps, ln_s,
                     ln_c, ln_out, epilogue, false, stream);
}

extern "C" int zk_gemm_f16_ln_frag(const void *A, const void *W, void *C, int64_t M, int64_t N,
                                   int64_t K, int64_t lda, int64_t ldw, const float *ln_part,
                                   float ln_eps, const float *ln_s, const float *ln_c,
                                   float *ln_out, void *stream) {
  const char *who = "zk_gemm_f16_ln_frag";
  if (N % 64) return fail(ZK_ERR_UNSUPPORTED, "%s: N must be a multiple of 64", who);
  return gemm_f16_ln(who, A, W, C, M, N, K, lda, ldw, N, ln_part, ln_eps, ln_s, ln_c, ln_out,
                     ZK_EPI_BIAS_GELU_ERF, true, stream);
}

// Shape / operand checks shared by the int8 entry points.
static int check_i8(const char *who, const int8_t *A, const int8_t *W, const void *C, int64_t M,
                    int64_t N, int64_t K, int64_t lda, int64_t ldw, int64_t ldc, int epilogue) {
  int st = check_dims(who, M, N, K);
  if (st) return st;
  if (M == 0 || N == 0) return ZK_OK;
  if (!A || !W || !C) return fail(ZK_ERR_INVALID, "%s: null pointer", who);
  if (epilogue < ZK_EPI_NONE || epilogue > ZK_EPI_BIAS_RELU)
    return fail(ZK_ERR_INVALID, "%s: bad epilogue %d", who, epilogue);
  if (lda < K || ldw < K || ldc < N)
    return fail(ZK_ERR_INVALID, "%s: leading dimension too small", who);
  if (K % 16 || lda % 16 || ldw % 16 || !aligned16(A) || !aligned16(W))
    return fail(ZK_ERR_UNSUPPORTED,
                "%s: K, lda, ldw must be multiples of 16 and A, W 16-byte aligned", who);
  if (K == 0) return fail(ZK_ERR_UNSUPPORTED, "%s: K == 0", who);
  // |acc| <= 128 * 128 * K, which reaches 2^31 (int32 overflow) at K = 131072
  if (K >= 131072)
    return fail(ZK_ERR_UNSUPPORTED, "%s: K >= 131072 could overflow int32 accumulators", who);
  return check_span(who, lda, ldw, K, 1);
}

extern "C" int zk_gemm_i8(const int8_t *A, const int8_t *W, void *C, int64_t M,
                          int64_t N, int64_t K, int64_t lda, int64_t ldw,
                          int64_t ldc, float s_x, const float *s_w,
                          const void *bias, const void *residual, int64_t ldr,
                          int epilogue, int out_dtype, void *stream) {
  int st = check_i8("zk_gemm_i8", A, W, C, M, N, K, lda, ldw, ldc, epilogue);
  if (st || M == 0 || N == 0) return st;
  hipStream_t s = as_stream(stream);
  GemmParams p{A, W, C, (int)M, (int)N, (int)K, lda, ldw, ldc, bias, residual, ldr, s_x, s_w, 0};
  if (out_dtype == ZK_I32) {
    if (epilogue != ZK_EPI_NONE)
      return fail(ZK_ERR_INVALID, "zk_gemm_i8: int32 output takes no epilogue");
    return launched(launch_mfma<I8Op, int32_t, false>(p, ZK_EPI_NONE, s), "zk_gemm_i8",
                    ZK_EPI_NONE);
  }
  if (!s_w) return fail(ZK_ERR_INVALID, "zk_gemm_i8: dequantised output needs s_w");
  if (!(s_x > 0.f)) return fail(ZK_ERR_INVALID, "zk_gemm_i8: s_x must be > 0");
  if (epilogue != ZK_EPI_NONE && !bias)
    return fail(ZK_ERR_INVALID, "zk_gemm_i8: epilogue needs a bias");
  if (epilogue == ZK_EPI_BIAS_RESIDUAL && (!residual || ldr < N))
    return fail(ZK_ERR_INVALID, "zk_gemm_i8: residual epilogue needs residual and ldr >= N");
  bool ok;
  if (out_dtype == ZK_F16) ok = launch_mfma<I8Op, f16, true>(p, epilogue, s);
  else if (out_dtype == ZK_F32) ok = launch_mfma<I8Op, float, true>(p, epilogue, s);
  else return fail(ZK_ERR_UNSUPPORTED, "zk_gemm_i8: out_dtype %d not supported", out_dtype);
  return launched(ok, "zk_gemm_i8", epilogue);
}

extern "C" int zk_gemm_i8_requant(const int8_t *A, const int8_t *W, int8_t *Q, int64_t M,
                                  int64_t N, int64_t K, int64_t lda, int64_t ldw,
                                  int64_t ldq, float s_x, const float *s_w,
                                  const void *bias, int epilogue, float s_out,
                                  void *stream) {
  int st = check_i8("zk_gemm_i8_requant", A, W, Q, M, N, K, lda, ldw, ldq, epilogue);
  if (st || M == 0 || N == 0) return st;
  if (epilogue == ZK_EPI_BIAS_RESIDUAL)
    return fail(ZK_ERR_INVALID, "zk_gemm_i8_requant: no residual epilogue for int8 output");
  if (!s_w) return fail(ZK_ERR_INVALID, "zk_gemm_i8_requant: s_w is required");
  if (!(s_x > 0.f) || !(s_out > 0.f))
    return fail(ZK_ERR_INVALID, "zk_gemm_i8_requant: s_x and s_out must be > 0");
  if (epilogue != ZK_EPI_NONE && !bias)
    return fail(ZK_ERR_INVALID, "zk_gemm_i8_requant: epilogue needs a bias");
  GemmParams p{A, W, Q, (int)M, (int)N, (int)K, lda, ldw, ldq, bias, nullptr, 0, s_x, s_w, 0};
  p.s_q = s_out;
  return launched(launch_mfma<I8Op, int8_t, true>(p, epilogue, as_stream(stream)),
                  "zk_gemm_i8_requant", epilogue);
}

extern "C" int zk_gemm_i8_requant_frag(const int8_t *A, const int8_t *W, int8_t *Q, int64_t M,
                                       int64_t N, int64_t K, int64_t lda, int64_t ldw,
                                       float s_x, const float *s_w, const void *bias,
                                       int epilogue, float s_out, void *stream) {
  const char *who = "zk_gemm_i8_requant_frag";
  int st = check_i8(who, A, W, Q, M, N, K, lda, ldw, N, epilogue);
  if (st || M == 0 || N == 0) return st;
  if (N % 128) return fail(ZK_ERR_UNSUPPORTED, "%s: N must be a multiple of 128", who);
  if (epilogue == ZK_EPI_BIAS_RESIDUAL)
    return fail(ZK_ERR_INVALID, "%s: no residual epilogue for int8 output", who);
  if (!s_w) return fail(ZK_ERR_INVALID, "%s: s_w is required", who);
  if (!(s_x > 0.f) || !(s_out > 0.f)) return fail(ZK_ERR_INVALID, "%s: s_x and s_out must be > 0", who);
  if (epilogue != ZK_EPI_NONE && !bias) return fail(ZK_ERR_INVALID, "%s: epilogue needs a bias", who);
  if (!aligned16(Q)) return fail(ZK_ERR_UNSUPPORTED, "%s: Q must be 16-byte aligned", who);
  GemmParams p{A, W, Q, (int)M, (int)N, (int)K, lda, ldw, N, bias, nullptr, 0, s_x, s_w, 0};
  p.s_q = s_out;
  p.c_pk = 1;
  // every 32x32-MFMA tile (0, 1, 4, 5) has the fragment-ordered store; the
  // 16x16 ones (2, 3) give way to the 128x96 tile
  int cfg = pick_cfg(p.M, p.N, p.K);
  if (cfg == 2 || cfg == 3) cfg = 4;
  return launched(launch_mfma<I8Op, int8_t, true>(p, epilogue, as_stream(stream), cfg), who,
                  epilogue);
}

extern "C" int zk_gemm_i8_res_stats_frag(const int8_t *A, const int8_t *W, void *C, int64_t M,
                                         int64_t N, int64_t K, int64_t ldw, int64_t ldc,
                                         float s_x, const float *s_w, const void *bias,
                                         const void *res, int64_t ldr, const float *res_ln,
                                         const void *res_gamma, const void *res_beta,
                                         float *part_out, void *stream) {
  const char *who = "zk_gemm_i8_res_stats_frag";
  int st = check_i8(who, A, W, C, M, N, K, K, ldw, ldc, ZK_EPI_BIAS);
  if (st || M == 0 || N == 0) return st;
  if (K % 128) return fail(ZK_ERR_UNSUPPORTED, "%s: K must be a multiple of 128", who);
  if (!aligned16(A)) return fail(ZK_ERR_UNSUPPORTED, "%s: A must be 16-byte aligned", who);
  if (!s_w || !(s_x > 0.f)) return fail(ZK_ERR_INVALID, "%s: s_w and s_x > 0 are required", who);
  if (ldc % 8 || !aligned16(C))
    return fail(ZK_ERR_UNSUPPORTED, "%s: ldc must be a multiple of 8 and C 16-byte aligned", who);
  GemmParams p{A, W, C, (int)M, (int)N, (int)K, K, ldw, ldc, bias, res, ldr, s_x, s_w, 0};
  p.a_pk = A;
  return res_stats_run<I8Op, true>(who, p, res_ln, res_gamma, res_beta, part_out, stream);
}

// Epilogue of the SIMT fp32 path, in place on C: the same operations, in the
// same order, as the MFMA kernel's epilogue.
template <int EPI>
__global__ __launch_bounds__(256) void f32_epilogue_kernel(float *__restrict__ C, int64_t ldc,
                                                           int64_t M, int64_t N,
                                                           const float *__restrict__ bias,
                                                           const float *__restrict__ res,
                                                           int64_t ldr) {
  const int64_t total = M * N, stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / N, c = i % N;
    float v = epilogue<EPI>(C[r * ldc + c], bias[c]);
    if (EPI == ZK_EPI_BIAS_RESIDUAL) v += res[r * ldr + c];
    C[r * ldc + c] = v;
  }
}

static int gemm_f32_impl(const float *A, const float *B, float *C, int64_t M, int64_t N,
                         int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int trans_b, void *ws,
                         int64_t ws_bytes, void *stream, const float *bias = nullptr,
                         const float *res = nullptr, int64_t ldr = 0, int epi = ZK_EPI_NONE,
                         const char *who = "zk_gemm_f32") {
  int st = check_dims(who, M, N, K);
  if (st) return st;
  if (M == 0 || N == 0) return ZK_OK;
  if (!A || !B || !C) return fail(ZK_ERR_INVALID, "%s: null pointer", who);
  if (lda < K || ldc < N || (trans_b ? ldb < K : ldb < N))
    return fail(ZK_ERR_INVALID, "%s: leading dimension too small", who);
  hipStream_t s = as_stream(stream);
  // W[N,K] operand with 16-byte rows: the MFMA kernel (fp32 matrix-core
  // products, fp32 accumulation); buffer offsets of a 256-row tile must fit
  // in 31 bits.
  if (trans_b && K > 0 && K % 4 == 0 && lda % 4 == 0 && ldb % 4 == 0 && aligned16(A) &&
      aligned16(B) && 255 * (lda + ldb) * 4 + 2 * K * 4 < 0x7ffffff0LL) {
    GemmParams p{A, B, C, (int)M, (int)N, (int)K, lda, ldb, ldc, bias, res, ldr, 1.f, nullptr, 0};
    const SplitPlan sp = plan_split(M, N, K, 4);
    bool ok;
    if (ws && sp.splits > 1 && ws_bytes >= split_ws_bytes(M, N, sp) && aligned16(ws))
      ok = launch_split<F32Op, float>(p, epi, sp, (float *)ws, s);
    else
      ok = launch_mfma<F32Op, float, false>(p, epi, s);
    return launched(ok, who, epi);
  }
  if ((M + 63) / 64 > 65535) return fail(ZK_ERR_UNSUPPORTED, "zk_gemm_f32: M too large");
  dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
  if (trans_b)
    gemm_f32_kernel<true><<<grid, 256, 0, s>>>(A, B, C, (int)M, (int)N, (int)K, lda, ldb, ldc);
  else
    gemm_f32_kernel<false><<<grid, 256, 0, s>>>(A, B, C, (int)M, (int)N, (int)K, lda, ldb, ldc);
  if (epi != ZK_EPI_NONE) {
    int64_t g = (M * N + 255) / 256;
    if (g > 4096) g = 4096;
#define ZK_E(E) f32_epilogue_kernel<E><<<(unsigned)g, 256, 0, s>>>(C, ldc, M, N, bias, res, ldr)
    switch (epi) {
      case ZK_EPI_BIAS: ZK_E(ZK_EPI_BIAS); break;
      case ZK_EPI_BIAS_GELU_ERF: ZK_E(ZK_EPI_BIAS_GELU_ERF); break;
      case ZK_EPI_BIAS_GELU_TANH: ZK_E(ZK_EPI_BIAS_GELU_TANH); break;
      case ZK_EPI_BIAS_RESIDUAL: ZK_E(ZK_EPI_BIAS_RESIDUAL); break;
      case ZK_EPI_BIAS_RELU: ZK_E(ZK_EPI_BIAS_RELU); break;
    }
#undef ZK_E
  }
  return check_launch(who);
}

extern "C" int zk_gemm_f32(const float *A, const float *B, float *C, int64_t M,
                           int64_t N, int64_t K, int64_t lda, int64_t ldb,
                           int64_t ldc, int trans_b, void *stream) {
  return gemm_f32_impl(A, B, C, M, N, K, lda, ldb, ldc, trans_b, nullptr, 0, stream);
}

extern "C" int zk_gemm_f32_ws(const float *A, const float *B, float *C, int64_t M, int64_t N,
                              int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int trans_b,
                              void *workspace, int64_t ws_bytes, void *stream) {
  if (ws_bytes < 0) return fail(ZK_ERR_INVALID, "zk_gemm_f32_ws: negative workspace size");
  return gemm_f32_impl(A, B, C, M, N, K, lda, ldb, ldc, trans_b, workspace, ws_bytes, stream);
}

extern "C" int zk_linear_f32(const float *X, const float *W, float *Y, int64_t M, int64_t N,
                             int64_t K, int64_t ldx, int64_t ldw, int64_t ldy,
                             const float *bias, const float *residual, int64_t ldr,
                             int epilogue, void *workspace, int64_t ws_bytes, void *stream) {
  if (ws_bytes < 0) return fail(ZK_ERR_INVALID, "zk_linear_f32: negative workspace size");
  if (epilogue < ZK_EPI_NONE || epilogue > ZK_EPI_BIAS_RELU)
    return fail(ZK_ERR_INVALID, "zk_linear_f32: bad epilogue %d", epilogue);
  if (epilogue != ZK_EPI_NONE && !bias)
    return fail(ZK_ERR_INVALID, "zk_linear_f32: epilogue needs a bias");
  if (epilogue == ZK_EPI_BIAS_RESIDUAL && (!residual || ldr < N))
    return fail(ZK_ERR_INVALID, "zk_linear_f32: residual epilogue needs residual and ldr >= N");
  return gemm_f32_impl(X, W, Y, M, N, K, ldx, ldw, ldy, 1, workspace, ws_bytes, stream, bias,
                       residual, ldr, epilogue, "zk_linear_f32");
}

extern "C" int64_t zk_gemm_workspace_size(int64_t M, int64_t N, int64_t K, int dtype) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  if (dtype == ZK_F16) return split_ws_bytes(M, N, plan_split(M, N, K, 2));
  if (dtype == ZK_F32) return split_ws_bytes(M, N, plan_split(M, N, K, 4));
  return 0;
}

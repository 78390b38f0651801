// Flash-attention forward (non-causal, optional key-padding mask).
//
// fp16 path (MFMA). A workgroup of NW wavefronts owns NW*32 query rows of
// one (batch, head); every wavefront owns 32 of them. Keys are walked in
// tiles of 64: K and V are staged in LDS as [key][d] with 16-byte stores (or
// DMA'd there, fa_fwd_f16_ring_kernel); the V^T fragments of the P.V product
// come out of the transposing LDS read.
// The wavefront computes S^T = K . Q^T with 32x32x16 MFMAs, so each lane
// ends up holding 32 keys of ONE query column (lane % 32): the row max and
// row sum of the online softmax are then a register loop plus a single
// swap with lane ^ 32, and the per-query rescale factor is lane-uniform.
// The exponentiated scores, rounded to fp16, are already laid out as the B
// operand of O^T += V^T . P^T, so P never leaves registers. Statistics and
// accumulation are fp32; exp2 with the softmax scale folded into log2(e).
// Key tiles at or beyond the sequence's valid length are never loaded; keys
// >= valid length inside the last tile get probability exactly 0, and a
// query with no valid key produces 0 (mask rule of the reference's masked
// attention primitive).
//
// For D = 64 and at most 128 queries, fa_fwd_f16_q16_kernel below does the
// same arithmetic with 16 queries per wavefront on 16x16x32 MFMAs.
//
// fp32 path (SIMT): D/32 lanes per query, each holding 32 dims of q and of
// the output accumulator; K/V tiles in LDS are read as broadcasts.
#include "zk_attn_tile.hpp"

namespace zk {

// (query block, head, batch) of this workgroup. The gridDim.x query blocks of
// one (batch, head) read the same K and V. Workgroups go to the 8 XCDs
// round-robin by linear id, so when B*H is a multiple of 8 the blocks of one
// head are given ids 8 apart: they run on one XCD and share its L2. At b32
// s128 this cut the L2-miss reads from 31.5 MB to 18.9 MB (Q, K and V once).
struct AttnTile {
  int qb, h, b;
};
__device__ __forceinline__ AttnTile attn_tile() {
  const int64_t gx = gridDim.x, nh = gridDim.y, nbh = nh * gridDim.z;
  if (gx == 1 || nbh % 8 != 0) return {(int)blockIdx.x, (int)blockIdx.y, (int)blockIdx.z};
  const int64_t bid = blockIdx.x + gx * (blockIdx.y + nh * blockIdx.z);
  const int64_t grp = bid / (8 * gx), rem = bid % (8 * gx);
  const int64_t bh = grp * 8 + rem % 8;
  return {(int)(rem / 8), (int)(bh % nh), (int)(bh / nh)};
}

// The 16-query kernel's transposing V read gives each 16-lane group 4 rows x
// 2 chunks (group g: rows 4g .. 4g+3), and the LDS serves a 64-bit read in
// two passes, one pairing the groups (0, 2) and (1, 3). kv_swz puts rows r
// and r + 8 in the same slots, which costs each such read an extra pass.
// kv_swz16 keeps the two chunks of a row in one aligned slot pair 2h, 2h+1
// with h distinct over the even (and the odd) rows of groups {0,1}, {2,3},
// {0,2} and {1,3}, and (h, low bit) distinct over all 16 rows for the K
// fragment reads. LDS bank-conflict cycles of the b32 s128 launch: 1.97e5
// with kv_swz, 0 with kv_swz16 (the encoder's time is unchanged).
__device__ __forceinline__ int kv_swz16(int r) {
  return 2 * (((r >> 1) & 3) ^ ((r >> 2) & 2)) + ((r >> 3) & 1);
}

// PAD: the stored head_dim p.D (a multiple of 8) is below the compiled D;
// dims >= p.D of Q, K and V are read as zeros (they add nothing to Q.K^T and
// produce output columns that are not stored).
// MASK: p.mask is applied on top of the valid lengths. A tile can then be
// fully masked for a query that has seen no valid key yet (running max still
// -inf); the rescale factor and the exponent are guarded for that case.
template <int D, int NW, bool PAD = false, bool MASK = false>
__global__ __launch_bounds__(NW * 64) void fa_fwd_f16_kernel(AttnParams p) {
  constexpr int KT = 64;
  constexpr int NT = NW * 64;
  constexpr bool SWZ = D == 64;  // swizzled unpadded rows (else padded rows)
  constexpr int KLD = SWZ ? D : D + 8;  // K and V tile row pitch (halves)
  constexpr int DV = D / 8;    // 16-byte vectors per K/V row
  constexpr int PER = KT * DV / NT;
  static_assert(KT * DV % NT == 0, "tile/thread mismatch");
  __shared__ __attribute__((aligned(16))) f16 Ks[KT * KLD];
  __shared__ __attribute__((aligned(16))) f16 Vs[KT * KLD];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h32 = lane >> 5;
  const AttnTile tile = attn_tile();
  const int b = tile.b, h = tile.h;
  const int L = valid_len(p, b);
  const f16 *Qb = (const f16 *)p.Q + b * p.sq[0] + h * p.sq[1];
  const f16 *Kb = (const f16 *)p.K + b * p.sk[0] + h * p.sk[1];
  const f16 *Vb = (const f16 *)p.V + b * p.sv[0] + h * p.sv[1];
  f16 *Ob = (f16 *)p.O + b * p.so[0] + h * p.so[1];

  const int qrow = tile.qb * (NW * 32) + wave * 32 + (lane & 31);
  const bool qvalid = qrow < p.Sq;
  const uint8_t *mrow = MASK ? mask_row(p, b, h, qvalid ? qrow : 0) : nullptr;
  f16x8 qf[D / 16];
#pragma unroll
  for (int c = 0; c < D / 16; ++c)
    qf[c] = qvalid && (!PAD || c * 16 + h32 * 8 < p.D)
                ? *(const f16x8 *)(Qb + qrow * p.sq[2] + c * 16 + h32 * 8)
                : f16x8{0, 0, 0, 0, 0, 0, 0, 0};

  f32x16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
  float m = -__builtin_inff(), l = 0.f;

  const int ntiles = (L + KT - 1) / KT;
  f16x8 kr[PER], vr[PER];
  auto load_kv = [&](int t) {
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int idx = tid + v * NT;
      const int kk = t * KT + idx / DV;  // K: 16-byte vectors row-contiguous
      const bool in = kk < p.Sk && (!PAD || (idx % DV) * 8 < p.D);
      kr[v] = in ? *(const f16x8 *)(Kb + kk * p.sk[2] + (idx % DV) * 8)
                 : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
      // V like K (8 lanes per 128-byte row, coalesced)
      vr[v] = in ? *(const f16x8 *)(Vb + kk * p.sv[2] + (idx % DV) * 8)
                 : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
  };
  auto stash_kv = [&]() {
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int idx = tid + v * NT;
      const int row = idx / DV, ch = SWZ ? (idx % DV) ^ kv_swz(row) : idx % DV;
      *(f16x8 *)(Ks + row * KLD + ch * 8) = kr[v];
      *(f16x8 *)(Vs + row * KLD + ch * 8) = vr[v];
    }
  };

  if (ntiles > 0) load_kv(0);
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();  // every wavefront is done with the previous tile
    stash_kv();
    __syncthreads();
    if (t + 1 < ntiles) load_kv(t + 1);

    attn32_tile<D, SWZ, KLD, MASK>(Ks, Vs, qf, t, L, p.scale_log2, &p, mrow, lane, o, m, l);
  }

  if (qvalid) {
    const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (PAD && dt * 32 + 8 * g + 4 * h32 >= p.D) continue;
        f16x4 out;
#pragma unroll
        for (int j = 0; j < 4; ++j) out[j] = (f16)(o[dt][4 * g + j] * inv);
        *(f16x4 *)(Ob + qrow * p.so[2] + dt * 32 + 8 * g + 4 * h32) = out;
      }
  }
}

// fp16, D = 64, key-padding lengths only (no boolean mask): the arithmetic
// of fa_fwd_f16_kernel with 8 wavefronts of 32 queries, but K and V go
// global -> LDS by DMA (buffer_load ... lds, 16 bytes per lane, nothing
// staged in registers) into a ring of ST stages of one 64-key tile each
// (8 KB of K, then 8 KB of V), so that up to ST - 1 tiles are in flight
// while one is multiplied. One wavefront instruction moves 8 rows: wave w
// fills rows 8w .. 8w + 7 of the K and of the V tile, lane l landing in
// slot l % 8 of row 8w + l / 8, so it fetches the logical chunk whose
// kv_swz slot that is. Keys at or beyond Sk lie past the buffer's end and
// read as 0; keys in [valid length, Sk) are loaded and given probability 0,
// as in fa_fwd_f16_kernel. The host launches it only when every byte offset
// fits 31 bits. (A boolean mask is read from global memory inside the tile
// loop, and that load could only be waited for together with the DMA of the
// tiles in flight before it; fa_fwd_f16_kernel serves that case.)
template <int ST>
__global__ __launch_bounds__(512) void fa_fwd_f16_ring_kernel(AttnParams p) {
  constexpr int D = 64, NW = 8, KT = 64, TILE = KT * D * 2;
  __shared__ __attribute__((aligned(1024))) char ring[ST * 2 * TILE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h32 = lane >> 5;
  const AttnTile tile = attn_tile();
  const int b = tile.b, h = tile.h;
  const int L = valid_len(p, b);
  const f16 *Qb = (const f16 *)p.Q + b * p.sq[0] + h * p.sq[1];
  const f16 *Kb = (const f16 *)p.K + b * p.sk[0] + h * p.sk[1];
  const f16 *Vb = (const f16 *)p.V + b * p.sv[0] + h * p.sv[1];
  f16 *Ob = (f16 *)p.O + b * p.so[0] + h * p.so[1];

  const int qrow = tile.qb * (NW * 32) + wave * 32 + (lane & 31);
  const bool qvalid = qrow < p.Sq;
  f16x8 qf[D / 16];
#pragma unroll
  for (int c = 0; c < D / 16; ++c)
    qf[c] = qvalid ? *(const f16x8 *)(Qb + qrow * p.sq[2] + c * 16 + h32 * 8)
                   : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  f32x16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
  float m = -__builtin_inff(), l = 0.f;

  const int ntiles = (L + KT - 1) / KT;
  const int rsk = (int)(p.sk[2] * 2), rsv = (int)(p.sv[2] * 2);  // row strides, bytes
  const __amdgpu_buffer_rsrc_t rK = __builtin_amdgcn_make_buffer_rsrc(
      (void *)Kb, (short)0, (p.Sk - 1) * rsk + D * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t rV = __builtin_amdgcn_make_buffer_rsrc(
      (void *)Vb, (short)0, (p.Sk - 1) * rsv + D * 2, 0x00020000);
  const int trow = wave * 8 + (lane >> 3), chunk = (lane & 7) ^ kv_swz(trow);
  const int offK = trow * rsk + chunk * 16, offV = trow * rsv + chunk * 16;
  // Two instructions per tile and wavefront. The host compilation pass sees
  // an empty statement (its check of this builtin with a run-time offset
  // rejects the kernel).
  auto issue = [&](int t, int stage) {
#if defined(__HIP_DEVICE_COMPILE__)
    char *ks = ring + stage * 2 * TILE;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rK, ZK_LDS(ks + wave * 1024), 16,
                                             offK + t * KT * rsk, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rV, ZK_LDS(ks + TILE + wave * 1024), 16,
                                             offV + t * KT * rsv, 0, 0, 0);
#else
    (void)t, (void)stage;
#endif
  };
#pragma unroll
  for (int s = 0; s < ST; ++s)
    if (s < ntiles) issue(s, s);
  if (ntiles > 0) {
    wait_slices<ST - 1, 2>(ntiles - 1);
    lds_barrier();
  }
  int stage = 0;
  for (int t = 0; t < ntiles; ++t) {
    const char *ks = ring + stage * 2 * TILE;
    attn32_tile<D, true, D, false>((const f16 *)ks, (const f16 *)(ks + TILE), qf, t, L,
                                   p.scale_log2, &p, nullptr, lane, o, m, l);
    if (t + 1 < ntiles) {
      // tile t + 1 has landed (up to ST - 2 younger tiles still in flight),
      // and after the barrier every wavefront is done reading tile t, whose
      // stage then receives tile t + ST
      wait_slices<ST - 2, 2>(ntiles - 2 - t);
      lds_barrier();
      if (t + ST < ntiles) issue(t + ST, stage);
      stage = stage + 1 == ST ? 0 : stage + 1;
    }
  }

  if (qvalid) {
    const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f16x4 out;
#pragma unroll
        for (int j = 0; j < 4; ++j) out[j] = (f16)(o[dt][4 * g + j] * inv);
        *(f16x4 *)(Ob + qrow * p.so[2] + dt * 32 + 8 * g + 4 * h32) = out;
      }
  }
}

// fp16, D = 64, 16 queries per wavefront on 16x16x32 MFMAs, NW wavefronts
// per workgroup. Same arithmetic as fa_fwd_f16_kernel (fp32 statistics, exp2
// with the scale folded in, lazy rescaling, P rounded to fp16), with half
// the per-wavefront dependency chain and twice the wavefronts.
// S^T = K . Q^T: lane l supplies K[key 16 kb + l%16][dims 8 (l/16) + 32 ks ..]
// and Q[query l%16][same dims], and receives S^T[16 kb + 4 (l/16) + r][l%16].
// O^T += V^T . P^T over 32 keys per step: k-slot 8 g + j (g = l / 16) is key
// 4 g + j for j < 4 and 16 + 4 g + (j - 4) otherwise, so the B operand is the
// lane's own probabilities of key blocks 2 st and 2 st + 1, and the V^T
// operand comes from two transposing reads 16 keys apart.
template <int NW, int TPS = 1, bool MASK = false>
__global__ __launch_bounds__(NW * 64) void fa_fwd_f16_q16_kernel(AttnParams p) {
  constexpr int D = 64, KT = 64, NT = NW * 64, DV = D / 8;
  constexpr int PER = TPS * KT * DV / NT;  // TPS key tiles per LDS stage
  static_assert(TPS * KT * DV % NT == 0 && PER >= 1, "tile/thread mismatch");
  __shared__ __attribute__((aligned(16))) f16 Ks[TPS * KT * D];
  __shared__ __attribute__((aligned(16))) f16 Vs[TPS * KT * D];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const AttnTile tile = attn_tile();
  const int b = tile.b, h = tile.h;
  const int L = valid_len(p, b);
  const f16 *Qb = (const f16 *)p.Q + b * p.sq[0] + h * p.sq[1];
  const f16 *Kb = (const f16 *)p.K + b * p.sk[0] + h * p.sk[1];
  const f16 *Vb = (const f16 *)p.V + b * p.sv[0] + h * p.sv[1];
  f16 *Ob = (f16 *)p.O + b * p.so[0] + h * p.so[1];

  const int qrow = tile.qb * (NW * 16) + wave * 16 + c16;
  const bool qvalid = qrow < p.Sq;
  const uint8_t *mrow = MASK ? mask_row(p, b, h, qvalid ? qrow : 0) : nullptr;
  f16x8 qf[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
    qf[ks] = qvalid ? *(const f16x8 *)(Qb + qrow * p.sq[2] + 32 * ks + 8 * g)
                    : f16x8{0, 0, 0, 0, 0, 0, 0, 0};

  f32x4 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -__builtin_inff(), l = 0.f;

  const int ntiles = (L + KT - 1) / KT;
  const int nstages = (ntiles + TPS - 1) / TPS;
  f16x8 kr[PER], vr[PER];
  auto load_kv = [&](int stg) {
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int idx = tid + v * NT;
      const int kk = stg * TPS * KT + idx / DV;
      kr[v] = kk < p.Sk ? *(const f16x8 *)(Kb + kk * p.sk[2] + (idx % DV) * 8)
                        : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
      vr[v] = kk < p.Sk ? *(const f16x8 *)(Vb + kk * p.sv[2] + (idx % DV) * 8)
                        : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
  };
  auto stash_kv = [&]() {
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int idx = tid + v * NT;
      const int row = idx / DV, ch = (idx % DV) ^ kv_swz16(idx / DV);
      *(f16x8 *)(Ks + row * D + ch * 8) = kr[v];
      *(f16x8 *)(Vs + row * D + ch * 8) = vr[v];
    }
  };
  // V^T source address of this lane: key 4 g + l%16 / 4 (+ 32 st, + 16),
  // dims 16 db + 4 (l % 4); with the swizzle, chunk 2 db + (l%4)/2 of a row
  // r is in slot chunk ^ kv_swz16(r), and kv_swz16 ignores the +32 st / +16.
  const int r0 = 4 * g + (c16 >> 2);
  const int fv = kv_swz16(r0), vhalf = (c16 & 3) >> 1, vin = 4 * (c16 & 1);

  if (nstages > 0) load_kv(0);
  for (int stg = 0; stg < nstages; ++stg) {
    __syncthreads();
    stash_kv();
    __syncthreads();
    if (stg + 1 < nstages) load_kv(stg + 1);
    for (int sub = 0; sub < TPS; ++sub) {
      const int t = stg * TPS + sub;
      if (t >= ntiles) break;  // wave-uniform; no barrier in this loop
      const f16 *Kt = Ks + sub * KT * D;
      const f16 *Vt = Vs + sub * KT * D;

      f32x4 s4[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        s4[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int row = 16 * kb + c16;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const f16x8 kf = *(const f16x8 *)(Kt + row * D + (((4 * ks + g) ^ kv_swz16(row)) << 3));
          s4[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[ks], s4[kb], 0, 0, 0);
        }
      }
      if (t * KT + KT > L) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (t * KT + 16 * kb + 4 * g + r >= L) s4[kb][r] = -__builtin_inff();
      }
      if constexpr (MASK) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          const uint32_t m4 = mask4(p, mrow, t * KT + 16 * kb + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (((m4 >> (8 * r)) & 0xffu) == 0) s4[kb][r] = -__builtin_inff();
        }
      }
      float tmax = -__builtin_inff();
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
        tmax = smax(smax(tmax, s4[kb][0]), smax(s4[kb][1], smax(s4[kb][2], s4[kb][3])));
      const auto smax_op = [](float a, float b) { return smax(a, b); };
      tmax = bfly<16>(tmax, smax_op);
      // finite unless MASK (without a mask, key t*KT < L is valid)
      tmax = bfly<32>(tmax, smax_op) * p.scale_log2;
      if (__builtin_amdgcn_ballot_w64(tmax > m + 8.0f) != 0) {
        const float m_new = fmaxf(m, tmax);
        const float alpha = MASK && m_new == -__builtin_inff() ? 1.0f
                                                               : __builtin_amdgcn_exp2f(m - m_new);
        m = m_new;
        l *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int r = 0; r < 4; ++r) o[db][r] *= alpha;
      }
      const float mneg = MASK && m == -__builtin_inff() ? 0.0f : -m;
      float psum = 0.f;
      f16x8 pf[2];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float e = __builtin_amdgcn_exp2f(fmaf(s4[kb][r], p.scale_log2, mneg));
          psum += e;
          pf[kb >> 1][4 * (kb & 1) + r] = (f16)e;
        }
      psum = bfly<16>(psum, OpAdd{});
      psum = bfly<32>(psum, OpAdd{});
      l += psum;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const f16 *row = Vt + (32 * st + r0) * D + ((((2 * db + vhalf) ^ fv)) << 3) + vin;
          const f16x4 lo = lds_read_tr16(row);
          const f16x4 hi = lds_read_tr16(row + 16 * D);
          const f16x8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[st], o[db], 0, 0, 0);
        }
    }
  }

  if (qvalid) {
    const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      f16x4 out;
#pragma unroll
      for (int r = 0; r < 4; ++r) out[r] = (f16)(o[db][r] * inv);
      *(f16x4 *)(Ob + qrow * p.so[2] + 16 * db + 4 * g) = out;
    }
  }
}

// ---------------------------------------------------------------- fp32 ----
// Compiled for D in {32, 64, 128}; a stored head_dim p.D <= D is zero-padded
// (dims >= p.D are read as zeros and not stored).
template <int D>
__global__ __launch_bounds__(256) void fa_fwd_f32_kernel(AttnParams p) {
  constexpr int TPQ = D / 32;  // lanes per query
  constexpr int QPB = 256 / TPQ;
  constexpr int KT = 32;
  __shared__ float Ks[KT][D + 4];
  __shared__ float Vs[KT][D + 4];
  const int tid = threadIdx.x, part = tid % TPQ;
  const int b = blockIdx.z, h = blockIdx.y;
  const int L = valid_len(p, b);
  const float *Qb = (const float *)p.Q + b * p.sq[0] + h * p.sq[1];
  const float *Kb = (const float *)p.K + b * p.sk[0] + h * p.sk[1];
  const float *Vb = (const float *)p.V + b * p.sv[0] + h * p.sv[1];
  float *Ob = (float *)p.O + b * p.so[0] + h * p.so[1];
  const int qrow = blockIdx.x * QPB + tid / TPQ;
  const bool qvalid = qrow < p.Sq;
  const float scale = p.scale_log2;
  const uint8_t *mrow = p.mask ? mask_row(p, b, h, qvalid ? qrow : 0) : nullptr;

  float q[32], acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    q[i] = qvalid && part * 32 + i < p.D ? Qb[qrow * p.sq[2] + part * 32 + i] : 0.f;
    acc[i] = 0.f;
  }
  float m = -__builtin_inff(), l = 0.f;
  const int ntiles = (L + KT - 1) / KT;
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();
    for (int idx = tid; idx < KT * D; idx += 256) {
      const int kk = idx / D, d = idx % D, key = t * KT + kk;
      const bool in = key < p.Sk && d < p.D;
      Ks[kk][d] = in ? Kb[key * p.sk[2] + d] : 0.f;
      Vs[kk][d] = in ? Vb[key * p.sv[2] + d] : 0.f;
    }
    __syncthreads();
    float s[KT];
    float tmax = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 32; ++i) d = fmaf(q[i], Ks[j][part * 32 + i], d);
      if constexpr (TPQ >= 2) d = bfly<1>(d, OpAdd{});  // lanes of a query: a quad
      if constexpr (TPQ >= 4) d = bfly<2>(d, OpAdd{});
      const int key = t * KT + j;
      s[j] = key < L && (!mrow || mrow[key]) ? d * scale : -__builtin_inff();
      tmax = fmaxf(tmax, s[j]);
    }
    // a query whose keys so far are all masked keeps m = -inf: no rescale,
    // and exp2(-inf - 0) = 0 for its scores
    const float m_new = fmaxf(m, tmax);
    const float alpha = m_new == -__builtin_inff() ? 1.0f : exp2f(m - m_new);
    m = m_new;
    l *= alpha;
#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] *= alpha;
    const float mref = m == -__builtin_inff() ? 0.0f : m;
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      const float e = exp2f(s[j] - mref);
      l += e;
#pragma unroll
      for (int i = 0; i < 32; ++i) acc[i] = fmaf(e, Vs[j][part * 32 + i], acc[i]);
    }
  }
  if (qvalid) {
    const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i)
      if (part * 32 + i < p.D) Ob[qrow * p.so[2] + part * 32 + i] = acc[i] * inv;
  }
}

template <int D, bool PAD = false, bool MASK = false>
static void launch_f16_m(const AttnParams &p, hipStream_t s) {
  // 4 wavefronts x 32 queries per workgroup: at seq 128 one workgroup holds a
  // whole (batch, head), so K and V are read from HBM once.
  // Up to 128 queries (BERT s128), D = 64: 16-query wavefronts, 4 per
  // workgroup. The shorter per-wave chain and the doubled wave count win
  // where the kernel is latency-bound (encoder 0.5% faster per step at b32
  // s128); at s512 the 32-query kernel's lower LDS traffic per query wins.
  if constexpr (D == 64 && !PAD) {
    if (p.Sq <= 128) {
      // one 64-key tile per LDS stage, the next one loading under the
      // current one's MFMAs. Staging both tiles of a 128-key sequence at once
      // (TPS = 2) was 0.7% slower per encoder step, fp16 and INT8-FFN, in
      // both-order A/Bs on two boxes. A few (batch, head) pairs (one to
      // four 128-token sequences: 96 to 384 workgroups of one wavefront
      // instead of 24 to 96 of four) take one wavefront per workgroup, so
      // that more CUs share the work.
      const unsigned bh = (unsigned)p.H * (unsigned)p.B;
      if ((unsigned)((p.Sq + 63) / 64) * bh < 256) {
        dim3 grid((unsigned)((p.Sq + 15) / 16), (unsigned)p.H, (unsigned)p.B);
        fa_fwd_f16_q16_kernel<1, 1, MASK><<<grid, 64, 0, s>>>(p);
        return;
      }
      dim3 grid((unsigned)((p.Sq + 63) / 64), (unsigned)p.H, (unsigned)p.B);
      fa_fwd_f16_q16_kernel<4, 1, MASK><<<grid, 256, 0, s>>>(p);
      return;
    }
  }
  // From 384 queries on, D = 64 with lengths only: the same shape with K and
  // V DMA'd into a 3-stage ring (b32 s512, [B,H,S,D]: 43-45 -> 39.4-41.5 us,
  // bit-identical output; 2 and 4 stages level; with the encoder's strided
  // [B*S, 3H] layout level).
  // From 384 queries on (s512), 8 wavefronts (256 queries) per workgroup:
  // each staged K/V tile then serves twice the queries. The kernel is bound
  // by per-wave latency and occupancy (VALU 46% and matrix cores 19% busy at
  // 1.8 resident waves per SIMD), not by LDS bandwidth: at b32 s512 this
  // takes 42.2-42.9 us against 45.5-47.6 us with 4 wavefronts, while two
  // 32-query blocks per wavefront (half the LDS traffic per query, but 1-2
  // waves per SIMD) took 53-61 us. At 256 queries it would leave one
  // workgroup per (batch, head) and is slower (19.5 against 17.4 us).
  if constexpr (D == 64 && !PAD && !MASK) {
    const int64_t rs = 2 * (p.sk[2] > p.sv[2] ? p.sk[2] : p.sv[2]);
    if (p.Sq >= 384 && rs >= 0 && ((int64_t)p.Sk + 64) * rs + 128 < (int64_t(1) << 31)) {
      dim3 grid((unsigned)((p.Sq + 255) / 256), (unsigned)p.H, (unsigned)p.B);
      fa_fwd_f16_ring_kernel<3><<<grid, 512, 0, s>>>(p);
      return;
    }
  }
  if constexpr (D == 64) {
    if (p.Sq >= 384) {
      dim3 grid((unsigned)((p.Sq + 255) / 256), (unsigned)p.H, (unsigned)p.B);
      fa_fwd_f16_kernel<D, 8, PAD, MASK><<<grid, 512, 0, s>>>(p);
      return;
    }
  }
  if (p.Sq >= 128) {
    dim3 grid((unsigned)((p.Sq + 127) / 128), (unsigned)p.H, (unsigned)p.B);
    fa_fwd_f16_kernel<D, 4, PAD, MASK><<<grid, 256, 0, s>>>(p);
  } else {
    dim3 grid((unsigned)((p.Sq + 63) / 64), (unsigned)p.H, (unsigned)p.B);
    fa_fwd_f16_kernel<D, 2, PAD, MASK><<<grid, 128, 0, s>>>(p);
  }
}

template <int D, bool PAD = false>
static void launch_f16(const AttnParams &p, hipStream_t s) {
  if (p.mask) launch_f16_m<D, PAD, true>(p, s);
  else launch_f16_m<D, PAD, false>(p, s);
}

template <int D>
static void launch_f32(const AttnParams &p, hipStream_t s) {
  constexpr int QPB = 256 / (D / 32);
  dim3 grid((unsigned)((p.Sq + QPB - 1) / QPB), (unsigned)p.H, (unsigned)p.B);
  fa_fwd_f32_kernel<D><<<grid, 256, 0, s>>>(p);
}

}  // namespace zk

using namespace zk;

static int attn_impl(const char *who, const void *Q, const void *K, const void *V, void *O,
                     int64_t batch, int64_t heads, int64_t seq_q, int64_t seq_k,
                     int64_t head_dim, const int64_t *strides, const int32_t *valid_lens,
                     const uint8_t *mask, const int64_t *mask_strides, float scale, int dtype,
                     void *stream) {
  if (batch < 0 || heads < 0 || seq_q < 0 || seq_k < 0 || head_dim <= 0)
    return fail(ZK_ERR_INVALID, "%s: bad size", who);
  if (batch == 0 || heads == 0 || seq_q == 0) return ZK_OK;
  if (!Q || !K || !V || !O || !strides) return fail(ZK_ERR_INVALID, "%s: null pointer", who);
  if (batch > 65535 || heads > 65535 || seq_q > 0x7fffffff || seq_k > 0x7fffffff)
    return fail(ZK_ERR_UNSUPPORTED, "%s: size exceeds launch limits", who);
  // any head_dim up to 128, the reference's HEAD_DIM_MAX (flash_attention.cu:26)
  if (head_dim > 128)
    return fail(ZK_ERR_UNSUPPORTED, "%s: head_dim %lld > 128", who, (long long)head_dim);
  if (!(scale > 0.0f) || scale == __builtin_inff())
    return fail(ZK_ERR_INVALID, "%s: scale must be finite and > 0", who);
  for (int i = 0; i < 12; ++i)
    if (strides[i] < 0) return fail(ZK_ERR_INVALID, "%s: negative stride", who);
  AttnParams p;
  p.Q = Q; p.K = K; p.V = V; p.O = O;
  p.B = (int)batch; p.H = (int)heads; p.Sq = (int)seq_q; p.Sk = (int)seq_k;
  p.D = (int)head_dim;
  for (int i = 0; i < 3; ++i) {
    p.sq[i] = strides[i]; p.sk[i] = strides[3 + i];
    p.sv[i] = strides[6 + i]; p.so[i] = strides[9 + i];
  }
  p.valid_lens = valid_lens;
  p.mask = mask;
  p.sm[0] = p.sm[1] = p.sm[2] = 0;
  if (mask) {
    if (!mask_strides) return fail(ZK_ERR_INVALID, "%s: mask without strides", who);
    for (int i = 0; i < 3; ++i) {
      if (mask_strides[i] < 0) return fail(ZK_ERR_INVALID, "%s: negative mask stride", who);
      if (mask_strides[i] % 4)
        return fail(ZK_ERR_UNSUPPORTED, "%s: mask strides must be multiples of 4", who);
      p.sm[i] = mask_strides[i];
    }
    if (reinterpret_cast<uintptr_t>(mask) & 3u)
      return fail(ZK_ERR_UNSUPPORTED, "%s: mask must be 4-byte aligned", who);
  }
  p.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = as_stream(stream);
  if (dtype == ZK_F16) {
    for (int i = 0; i < 12; ++i)
      if (strides[i] % 8)
        return fail(ZK_ERR_UNSUPPORTED, "%s: fp16 strides must be multiples of 8", who);
    if (!aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(O))
      return fail(ZK_ERR_UNSUPPORTED, "%s: fp16 tensors must be 16-byte aligned", who);
    if (head_dim % 8)
      return fail(ZK_ERR_UNSUPPORTED, "%s: fp16 head_dim must be a multiple of 8 (got %lld)",
                  who, (long long)head_dim);
    // compiled widths 32 / 64 / 128; narrower head_dims are zero-padded
    if (head_dim == 32) launch_f16<32>(p, s);
    else if (head_dim == 64) launch_f16<64>(p, s);
    else if (head_dim == 128) launch_f16<128>(p, s);
    else if (head_dim < 32) launch_f16<32, true>(p, s);
    else if (head_dim < 64) launch_f16<64, true>(p, s);
    else launch_f16<128, true>(p, s);
  } else if (dtype == ZK_F32) {
    if (head_dim <= 32) launch_f32<32>(p, s);
    else if (head_dim <= 64) launch_f32<64>(p, s);
    else launch_f32<128>(p, s);
  } else {
    return fail(ZK_ERR_UNSUPPORTED, "%s: dtype %d not supported", who, dtype);
  }
  return check_launch(who);
}

extern "C" int zk_flash_attn_fwd(const void *Q, const void *K, const void *V, void *O,
                                 int64_t batch, int64_t heads, int64_t seq_q, int64_t seq_k,
                                 int64_t head_dim, const int64_t *strides,
                                 const int32_t *valid_lens, float scale, int dtype,
                                 void *stream) {
  return attn_impl("zk_flash_attn_fwd", Q, K, V, O, batch, heads, seq_q, seq_k, head_dim,
                   strides, valid_lens, nullptr, nullptr, scale, dtype, stream);
}

extern "C" int zk_flash_attn_fwd_masked(const void *Q, const void *K, const void *V, void *O,
                                        int64_t batch, int64_t heads, int64_t seq_q,
                                        int64_t seq_k, int64_t head_dim, const int64_t *strides,
                                        const int32_t *valid_lens, const uint8_t *mask,
                                        const int64_t *mask_strides, float scale, int dtype,
                                        void *stream) {
  if (!mask) return fail(ZK_ERR_INVALID, "zk_flash_attn_fwd_masked: null mask");
  return attn_impl("zk_flash_attn_fwd_masked", Q, K, V, O, batch, heads, seq_q, seq_k,
                   head_dim, strides, valid_lens, mask, mask_strides, scale, dtype, stream);
}

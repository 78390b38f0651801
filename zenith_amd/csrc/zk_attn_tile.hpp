// Device pieces shared by the flash-attention kernels and the fused
// QKV-projection + attention epilogue of the GEMM: parameters, masks, the
// score max, the transposing LDS read, the K/V swizzle, and one 64-key tile
// of the 32-query-per-wavefront online softmax.
#pragma once
#include "zk_common.hpp"

namespace zk {

struct AttnParams {
  const void *Q, *K, *V;
  void *O;
  int B, H, Sq, Sk;
  int D;  // head_dim as stored; kernels compiled for a wider width zero-pad to it
  int64_t sq[3], sk[3], sv[3], so[3];  // (batch, head, seq) strides
  const int32_t *valid_lens;
  // Optional boolean mask, one byte per (batch, head, query, key), nonzero =
  // attend; (batch, head, query) strides in bytes (0 broadcasts), keys
  // contiguous, every row 4-byte aligned (read 4 keys at a time).
  const uint8_t *mask;
  int64_t sm[3];
  float scale_log2;  // softmax scale * log2(e)
};

// The mask row of (b, h, q), and the 4 mask bytes of keys k0 .. k0 + 3 as one
// word (k0 a multiple of 4; keys >= Sk read as masked).
__device__ __forceinline__ const uint8_t *mask_row(const AttnParams &p, int b, int h, int q) {
  return p.mask + b * p.sm[0] + h * p.sm[1] + (int64_t)q * p.sm[2];
}
__device__ __forceinline__ uint32_t mask4(const AttnParams &p, const uint8_t *row, int k0) {
  return k0 < p.Sk ? *(const uint32_t *)(row + k0) : 0u;
}

__device__ __forceinline__ int valid_len(const AttnParams &p, int b) {
  if (!p.valid_lens) return p.Sk;
  int L = p.valid_lens[b];
  return L < 0 ? 0 : (L > p.Sk ? p.Sk : L);
}

// max(a, b) of scores that are never NaN, as v_med3(a, b, +inf). Chains of
// these compile to v_max3_f32 alone; fmaxf on MFMA results also makes a
// NaN-quieting copy of every operand (32 extra VALU instructions per
// 32 x 64 score tile of a wavefront).
__device__ __forceinline__ float smax(float a, float b) {
  return __builtin_amdgcn_fmed3f(a, b, __builtin_inff());
}

// ds_read_b64_tr_b16: 8 bytes per lane, transposed across each group of 16
// lanes (see its use below for the lane mapping).
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f16x4 lds_read_tr16(const f16 *p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4 *)(p));
  return __builtin_bit_cast(f16x4, v);
}

// D = 64 K/V tiles are stored as unpadded 128-byte rows with 16-byte chunk c
// of row r in slot c ^ kv_swz(r): a K fragment read (16 rows, one chunk per
// 16-lane group) and a transposing V read (4 rows x 4 chunks per 32 lanes)
// then both hit 64 distinct banks, which no uniform row padding achieves.
__device__ __forceinline__ int kv_swz(int r) {
  return ((r & 2) << 1) | ((r & 4) >> 1) | ((r >> 3) & 1);
}

// One 64-key tile of the 32-query wavefront (head dim D), in three phases
// that attn32_tile runs in a row; a kernel may interleave the phases of
// different wavefronts, each wavefront still running them in this order.
// Phase 1, attn32_qk: scores S^T = K.Q^T of the tile's two 32-key blocks
// from the K tile Kt (LDS, row pitch KLD halves, swizzled with kv_swz when
// SWZ); qf holds the wavefront's Q fragments.
template <int D, bool SWZ, int KLD>
__device__ __forceinline__ void attn32_qk(const f16 *__restrict__ Kt, const f16x8 (&qf)[D / 16],
                                          int lane, f32x16 (&s)[2]) {
  const int h32 = lane >> 5;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) s[kb][r] = 0.f;
  // the two key blocks' accumulation chains alternate, so consecutive
  // MFMAs never wait for each other's result
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
    const int kch = SWZ ? (2 * c + h32) ^ kv_swz(lane & 31) : 2 * c + h32;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const f16x8 kf = *(const f16x8 *)(Kt + (kb * 32 + (lane & 31)) * KLD + kch * 8);
      s[kb] = mfma32x32x16(kf, qf[c], s[kb]);
    }
  }
}

// (a, b) = (x of this lane, x of lane ^ 32) in some order, by one
// v_permlane32_swap (a VALU op, no LDS round trip as with __shfl_xor).
__device__ __forceinline__ void half_swap(float x, float &a, float &b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

// Phase 2, attn32_softmax: keys >= L and (MASK) masked keys set to -inf,
// online-softmax update of the running max m and sum l (lazy rescaling of
// o), and the probabilities as fp16 B fragments pf of the P.V product. t is
// the tile index (keys t*64 ..); mp / mrow are read only with MASK.
// It runs as two parts: attn32_softmax_max (masking, the tile max and the
// lazy rescale; returns the exponent offset) and attn32_softmax_exp (the
// probabilities and the row sum), so that a caller can place independent
// MFMAs among the second part's VALU work.
template <int D, bool MASK>
__device__ __forceinline__ float attn32_softmax_max(f32x16 (&s)[2], int t, int L,
                                                    float scale_log2, const AttnParams *mp,
                                                    const uint8_t *mrow, int lane,
                                                    f32x16 (&o)[D / 32], float &m, float &l) {
  constexpr int KT = 64;
  const int h32 = lane >> 5;
  // Tile max on the raw scores (the scale is positive), masking only the
  // tile that straddles the valid length.
  const bool partial = t * KT + KT > L;
  if (partial) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = t * KT + kb * 32 + 8 * (r >> 2) + 4 * h32 + (r & 3);
        if (key >= L) s[kb][r] = -__builtin_inff();
      }
  }
  if constexpr (MASK) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const uint32_t m4 = mask4(*mp, mrow, t * KT + kb * 32 + 8 * g4 + 4 * h32);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (((m4 >> (8 * j)) & 0xffu) == 0) s[kb][4 * g4 + j] = -__builtin_inff();
      }
  }
  float tmax = -__builtin_inff();
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) tmax = smax(tmax, s[kb][r]);
  // finite unless MASK (without a mask, key t*KT < L is valid)
  {
    float a, b;
    half_swap(tmax, a, b);
    tmax = smax(a, b) * scale_log2;
  }
  // Lazy rescaling: the reference point m (log2 units) only moves when the
  // tile max exceeds it by more than 8, so exp2(s - m) <= 256 always fits
  // fp16 and the accumulator is rescaled on a few tiles only. O / l is
  // independent of the reference point, so this is exact.
  if (__builtin_amdgcn_ballot_w64(tmax > m + 8.0f) != 0) {
    const float m_new = fmaxf(m, tmax);
    // 0 on the first tile; a query with no valid key yet keeps m = -inf
    const float alpha = MASK && m_new == -__builtin_inff() ? 1.0f
                                                           : __builtin_amdgcn_exp2f(m - m_new);
    m = m_new;
    l *= alpha;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
  }
  // with m = -inf every score of this query is -inf so far: exp2 gives 0
  return MASK && m == -__builtin_inff() ? 0.0f : -m;
}

// attn32_softmax_max without a mask and with the accumulator's rescale left
// to the caller: when resc (wavefront-uniform) is set, m has moved and l has
// been multiplied by alpha, and o must be multiplied by alpha before the
// next P.V product adds to it (so a P.V product of the previous tile may
// still run first, as it would have before this tile's rescale).
__device__ __forceinline__ float attn32_max_defer(f32x16 (&s)[2], int t, int L, float scale_log2,
                                                  int lane, float &m, float &l, float &alpha,
                                                  bool &resc) {
  constexpr int KT = 64;
  const int h32 = lane >> 5;
  if (t * KT + KT > L) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = t * KT + kb * 32 + 8 * (r >> 2) + 4 * h32 + (r & 3);
        if (key >= L) s[kb][r] = -__builtin_inff();
      }
  }
  float tmax = -__builtin_inff();
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) tmax = smax(tmax, s[kb][r]);
  {
    float a, b;
    half_swap(tmax, a, b);
    tmax = smax(a, b) * scale_log2;
  }
  resc = __builtin_amdgcn_ballot_w64(tmax > m + 8.0f) != 0;
  alpha = 1.0f;
  if (resc) {
    const float m_new = fmaxf(m, tmax);
    alpha = __builtin_amdgcn_exp2f(m - m_new);
    m = m_new;
    l *= alpha;
  }
  return -m;
}

template <int D>
__device__ __forceinline__ void attn32_softmax_exp(const f32x16 (&s)[2], float scale_log2,
                                                   float mneg, float &l, f16x8 (&pf)[2][2]) {
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      pf[kb][r >> 3][r & 7] = (f16)__builtin_amdgcn_exp2f(fmaf(s[kb][r], scale_log2, mneg));
  // the row sum of the probabilities as rounded to fp16 (the P the P.V
  // product uses), two at a time with v_dot2_f32_f16 against (1, 1)
  float psum = 0.f;
  const f16x2 one2 = {(f16)1.0f, (f16)1.0f};
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
      for (int e = 0; e < 8; e += 2)
        psum = __builtin_amdgcn_fdot2(f16x2{pf[kb][c2][e], pf[kb][c2][e + 1]}, one2, psum,
                                      false);
  {
    float a, b;
    half_swap(psum, a, b);
    l += a + b;  // the same sum in either order (fp32 addition commutes)
  }
}

template <int D, bool MASK>
__device__ __forceinline__ void attn32_softmax(f32x16 (&s)[2], int t, int L, float scale_log2,
                                               const AttnParams *mp, const uint8_t *mrow,
                                               int lane, f32x16 (&o)[D / 32], float &m,
                                               float &l, f16x8 (&pf)[2][2]) {
  const float mneg = attn32_softmax_max<D, MASK>(s, t, L, scale_log2, mp, mrow, lane, o, m, l);
  attn32_softmax_exp<D>(s, scale_log2, mneg, l, pf);
}

// Phase 3, attn32_pv: O^T[d][q] += V^T[d][key] . P^T[key][q] from the V
// tile Vt, 16 keys per MFMA. Lane-half h32, slot j of the P^T fragment
// holds key 16*c2 + 8*(j/4) + 4*h32 + j%4 of block kb; the V^T fragment
// (lane l: dim l % 32 of block dt, the same keys) comes from the row-major V
// tile through the transposing LDS read: in each group of 16 lanes, output
// lane i, slot j receives element i % 4 of the 4 elements read by source
// lane 4*j + i/4. Source lane s therefore reads key k0 + s/4, dims
// dbase + 4*(s%4), and output lane i gets dim dbase + i at keys k0 .. k0+3.
// (with SWZ: chunk ch of row r0 + 32 kb + 16 c2 sits in slot ch ^ kv_swz(r0),
// and of the row 8 further in slot ch ^ kv_swz(r0) ^ 1)
template <int D, bool SWZ, int KLD>
__device__ __forceinline__ void attn32_pv(const f16 *__restrict__ Vt, const f16x8 (&pf)[2][2],
                                          int lane, f32x16 (&o)[D / 32]) {
  const int grp = lane >> 4, sl = lane & 15;
  const int r0 = 4 * (grp >> 1) + (sl >> 2);
  const int fv = SWZ ? kv_swz(r0) : 0;
  const int vch = 2 * (grp & 1) + ((sl & 3) >> 1), vin = 4 * (sl & 1);
  // the D / 32 output blocks' accumulation chains alternate (each still
  // accumulates its key blocks in the same order)
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        const f16 *row = Vt + (r0 + kb * 32 + c2 * 16) * KLD;
        const int ch = 4 * dt + vch;
        const f16x4 lo = lds_read_tr16(row + (((ch ^ fv) << 3) + vin));
        const f16x4 hi = lds_read_tr16(row + 8 * KLD + (((ch ^ (SWZ ? fv ^ 1 : 0)) << 3) + vin));
        const f16x8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[dt] = mfma32x32x16(vf, pf[kb][c2], o[dt]);
      }
}

// The three phases of one tile in a row (Kt, Vt: the tile's K and V).
// Kt and Vt are restrict-qualified in every phase: the LDS reads through
// them then carry alias information, without which the compiler makes each
// transposing V read wait until every LDS DMA still in flight has landed
// (the callers order their DMA themselves, by explicit waits and barriers).
template <int D, bool SWZ, int KLD, bool MASK>
__device__ __forceinline__ void attn32_tile(const f16 *__restrict__ Kt, const f16 *__restrict__ Vt,
                                            const f16x8 (&qf)[D / 16], int t, int L,
                                            float scale_log2, const AttnParams *mp,
                                            const uint8_t *mrow, int lane, f32x16 (&o)[D / 32],
                                            float &m, float &l) {
  f32x16 s[2];
  attn32_qk<D, SWZ, KLD>(Kt, qf, lane, s);
  f16x8 pf[2][2];
  attn32_softmax<D, MASK>(s, t, L, scale_log2, mp, mrow, lane, o, m, l, pf);
  attn32_pv<D, SWZ, KLD>(Vt, pf, lane, o);
}

}  // namespace zk

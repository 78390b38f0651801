// Embedding lookups.
//
// zk_embedding: out[i, :] = table[ids[i], :] (the reference's embedding_f32).
// zk_bert_embeddings: the BERT input layer fused into one pass per token,
//   out[t, :] = LayerNorm(word[ids[t]] + pos[s + pos_offset] + type[tt[t]])
// with fp32 statistics (two-pass mean / variance over the summed row, which
// a wavefront keeps in registers). One wavefront per token; ids outside the
// table give a zero row (embedding) or are clamped out of the sum (BERT), so
// no id can send a load out of bounds.
#include "zk_common.hpp"

namespace zk {
namespace {

template <typename T> struct EV;
template <> struct EV<f16> { typedef f16x8 type; static constexpr int n = 8; };
template <> struct EV<float> { typedef f32x4 type; static constexpr int n = 4; };

constexpr int kEmbWaves = 4;

template <typename T, bool VEC>
__global__ __launch_bounds__(kEmbWaves * kWave) void embedding_kernel(
    const int32_t *__restrict__ ids, const T *__restrict__ table, T *__restrict__ out,
    int64_t n, int H, int64_t V) {
  typedef typename EV<T>::type Vt;
  constexpr int W = EV<T>::n;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t t = (int64_t)blockIdx.x * kEmbWaves + (threadIdx.x >> 6);
  if (t >= n) return;
  const int64_t id = ids[t];
  const bool ok = id >= 0 && id < V;
  if (VEC) {
    const Vt *src = reinterpret_cast<const Vt *>(table + (ok ? id : 0) * H);
    Vt *dst = reinterpret_cast<Vt *>(out + t * H);
    for (int j = lane; j < H / W; j += kWave) {
      Vt v = src[j];
      if (!ok) {
#pragma unroll
        for (int e = 0; e < W; ++e) v[e] = (T)0.f;
      }
      dst[j] = v;
    }
  } else {
    for (int j = lane; j < H; j += kWave) out[t * H + j] = ok ? table[id * H + j] : (T)0.f;
  }
}

// Row held in registers: MAXV vectors of W elements per lane.
template <typename T, int MAXV>
__global__ __launch_bounds__(kEmbWaves * kWave) void bert_embeddings_kernel(
    const int32_t *__restrict__ ids, const int32_t *__restrict__ types,
    const T *__restrict__ word, const T *__restrict__ pos, const T *__restrict__ type_tab,
    const T *__restrict__ gamma, const T *__restrict__ beta, T *__restrict__ out, int64_t n,
    int S, int H, int64_t V, int P, int NT, int pos_offset, float eps) {
  typedef typename EV<T>::type Vt;
  constexpr int W = EV<T>::n;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t t = (int64_t)blockIdx.x * kEmbWaves + (threadIdx.x >> 6);
  if (t >= n) return;  // whole wavefront
  const int64_t id = ids[t];
  const int s = (int)(t % S) + pos_offset;
  const int tt = types ? types[t] : 0;
  const bool wok = id >= 0 && id < V, pok = s >= 0 && s < P, tok = tt >= 0 && tt < NT;
  const Vt *wr = reinterpret_cast<const Vt *>(word + (wok ? id : 0) * H);
  const Vt *pr = reinterpret_cast<const Vt *>(pos + (int64_t)(pok ? s : 0) * H);
  const Vt *tr = reinterpret_cast<const Vt *>(type_tab + (int64_t)(tok ? tt : 0) * H);
  const int nvec = H / W;
  float v[MAXV][W];
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < MAXV; ++k) {
    const int j = lane + k * kWave;
    if (j < nvec) {
      const Vt a = wr[j], b = pr[j], c = tr[j];
#pragma unroll
      for (int e = 0; e < W; ++e) {
        const float f = (wok ? (float)a[e] : 0.f) + (pok ? (float)b[e] : 0.f) +
                        (tok ? (float)c[e] : 0.f);
        v[k][e] = f;
        sum += f;
      }
    } else {
#pragma unroll
      for (int e = 0; e < W; ++e) v[k][e] = 0.f;
    }
  }
  const float mean = wave_sum(sum) / (float)H;
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < MAXV; ++k) {
    if (lane + k * kWave < nvec) {
#pragma unroll
      for (int e = 0; e < W; ++e) {
        const float d = v[k][e] - mean;
        sq += d * d;
      }
    }
  }
  const float rstd = 1.0f / sqrtf(wave_sum(sq) / (float)H + eps);
  const Vt *gv = reinterpret_cast<const Vt *>(gamma);
  const Vt *bv = reinterpret_cast<const Vt *>(beta);
  Vt *dst = reinterpret_cast<Vt *>(out + t * H);
#pragma unroll
  for (int k = 0; k < MAXV; ++k) {
    const int j = lane + k * kWave;
    if (j < nvec) {
      const Vt g = gv[j], b = bv[j];
      Vt o;
#pragma unroll
      for (int e = 0; e < W; ++e) o[e] = (T)((v[k][e] - mean) * rstd * (float)g[e] + (float)b[e]);
      dst[j] = o;
    }
  }
}

template <typename T>
int bert_emb_impl(const int32_t *ids, const int32_t *types, const void *word, const void *pos,
                  const void *type_tab, const void *gamma, const void *beta, void *out,
                  int64_t B, int64_t S, int64_t H, int64_t V, int64_t P, int64_t NT,
                  int64_t pos_offset, float eps, hipStream_t s) {
  constexpr int W = EV<T>::n;
  if (H % W || !aligned16(word) || !aligned16(pos) || !aligned16(type_tab) ||
      !aligned16(gamma) || !aligned16(beta) || !aligned16(out))
    return fail(ZK_ERR_UNSUPPORTED,
                "zk_bert_embeddings: hidden must be a multiple of %d and tables 16-byte aligned", W);
  const int64_t nvec = H / W;
  const int64_t n = B * S;
  const unsigned g = (unsigned)((n + kEmbWaves - 1) / kEmbWaves);
#define ZK_E(MV)                                                                               \
  bert_embeddings_kernel<T, MV><<<g, kEmbWaves * kWave, 0, s>>>(                              \
      ids, types, (const T *)word, (const T *)pos, (const T *)type_tab, (const T *)gamma,     \
      (const T *)beta, (T *)out, n, (int)S, (int)H, V, (int)P, (int)NT, (int)pos_offset, eps)
  if (nvec <= kWave) ZK_E(1);
  else if (nvec <= 2 * kWave) ZK_E(2);
  else if (nvec <= 4 * kWave) ZK_E(4);
  else if (nvec <= 8 * kWave) ZK_E(8);
  else return fail(ZK_ERR_UNSUPPORTED, "zk_bert_embeddings: hidden %lld too large", (long long)H);
#undef ZK_E
  return check_launch("zk_bert_embeddings");
}

}  // namespace
}  // namespace zk

using namespace zk;

extern "C" int zk_embedding(const int32_t *ids, const void *table, void *out, int64_t n,
                            int64_t hidden, int64_t vocab, int dtype, void *stream) {
  if (n < 0 || hidden < 0 || vocab < 0) return fail(ZK_ERR_INVALID, "zk_embedding: negative size");
  if (n == 0 || hidden == 0) return ZK_OK;
  if (!ids || !table || !out) return fail(ZK_ERR_INVALID, "zk_embedding: null pointer");
  if (hidden > 0x7fffffff || (n + kEmbWaves - 1) / kEmbWaves > 0x7fffffff)
    return fail(ZK_ERR_UNSUPPORTED, "zk_embedding: size too large");
  const unsigned g = (unsigned)((n + kEmbWaves - 1) / kEmbWaves);
  hipStream_t s = as_stream(stream);
  const int H = (int)hidden;
  if (dtype == ZK_F32) {
    if (H % 4 == 0 && aligned16(table) && aligned16(out))
      embedding_kernel<float, true><<<g, kEmbWaves * kWave, 0, s>>>(ids, (const float *)table, (float *)out, n, H, vocab);
    else
      embedding_kernel<float, false><<<g, kEmbWaves * kWave, 0, s>>>(ids, (const float *)table, (float *)out, n, H, vocab);
  } else if (dtype == ZK_F16) {
    if (H % 8 == 0 && aligned16(table) && aligned16(out))
      embedding_kernel<f16, true><<<g, kEmbWaves * kWave, 0, s>>>(ids, (const f16 *)table, (f16 *)out, n, H, vocab);
    else
      embedding_kernel<f16, false><<<g, kEmbWaves * kWave, 0, s>>>(ids, (const f16 *)table, (f16 *)out, n, H, vocab);
  } else {
    return fail(ZK_ERR_UNSUPPORTED, "zk_embedding: dtype %d not supported", dtype);
  }
  return check_launch("zk_embedding");
}

extern "C" int zk_bert_embeddings(const int32_t *input_ids, const int32_t *token_type_ids,
                                  const void *word, const void *pos, const void *type_table,
                                  const void *gamma, const void *beta, void *out, int64_t batch,
                                  int64_t seq, int64_t hidden, int64_t vocab, int64_t max_pos,
                                  int64_t n_types, int64_t pos_offset, float eps, int dtype,
                                  void *stream) {
  if (batch < 0 || seq < 0 || hidden < 0 || vocab < 0 || max_pos < 0 || n_types < 0)
    return fail(ZK_ERR_INVALID, "zk_bert_embeddings: negative size");
  if (batch == 0 || seq == 0) return ZK_OK;
  if (!input_ids || !word || !pos || !type_table || !gamma || !beta || !out)
    return fail(ZK_ERR_INVALID, "zk_bert_embeddings: null pointer");
  if (hidden == 0 || vocab == 0 || max_pos == 0 || n_types == 0)
    return fail(ZK_ERR_INVALID, "zk_bert_embeddings: empty table");
  if (pos_offset < 0 || seq + pos_offset > max_pos)
    return fail(ZK_ERR_INVALID, "zk_bert_embeddings: positions exceed the position table");
  if (!(eps >= 0.f)) return fail(ZK_ERR_INVALID, "zk_bert_embeddings: eps must be >= 0");
  if (batch * seq / kEmbWaves > 0x7fffffff)
    return fail(ZK_ERR_UNSUPPORTED, "zk_bert_embeddings: too many tokens");
  hipStream_t s = as_stream(stream);
  if (dtype == ZK_F32)
    return bert_emb_impl<float>(input_ids, token_type_ids, word, pos, type_table, gamma, beta, out,
                                batch, seq, hidden, vocab, max_pos, n_types, pos_offset, eps, s);
  if (dtype == ZK_F16)
    return bert_emb_impl<f16>(input_ids, token_type_ids, word, pos, type_table, gamma, beta, out,
                              batch, seq, hidden, vocab, max_pos, n_types, pos_offset, eps, s);
  return fail(ZK_ERR_UNSUPPORTED, "zk_bert_embeddings: dtype %d not supported", dtype);
}

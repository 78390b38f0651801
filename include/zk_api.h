/*
 * zk_api.h - C ABI of libzenith_hip.so, the MI355X (gfx950) kernel library
 * behind the `zenith_cuda` drop-in (relu, gelu, layernorm, matmul,
 * flash_attention, wmma_matmul) and the fused BERT-encoder epilogues.
 *
 * Conventions (all entry points):
 *   - return int: ZK_OK (0) on success, a negative zk_status on failure;
 *     zk_last_error() then holds a message (thread-local).
 *   - every data pointer is a device pointer; sizes and leading dimensions
 *     are in elements; matrices are row-major.
 *   - the last argument is the HIP stream (hipStream_t passed as void*; NULL
 *     means the null stream). Launches are asynchronous; nothing is
 *     allocated and nothing synchronises inside the library.
 *   - no torch / C++ types cross this boundary.
 *
 * Each declaration cites the reference interface it replaces
 * (paths relative to the vibeswithkk/ZENITH source tree).
 */
#ifndef ZK_API_H
#define ZK_API_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  ZK_OK = 0,
  ZK_ERR_INVALID = -1,     /* bad pointer / negative size / bad enum value   */
  ZK_ERR_UNSUPPORTED = -2, /* valid request this library does not implement */
  ZK_ERR_HIP = -3          /* a HIP runtime call (launch) failed             */
} zk_status;

typedef enum { ZK_F32 = 0, ZK_F16 = 1, ZK_I8 = 2, ZK_I32 = 3 } zk_dtype;

/* GELU flavour: tanh approximation (reference CUDA kernels) or exact erf
 * (BERT / ONNX Gelu with Erf). */
typedef enum { ZK_GELU_TANH = 0, ZK_GELU_ERF = 1 } zk_gelu_mode;

/* GEMM epilogue applied to the fp32 (or dequantised int32) accumulator.
 * bias is a length-N vector of the output dtype (fp32 for fp32 output),
 * residual an [M, N] matrix of the output dtype with leading dim ldr. */
typedef enum {
  ZK_EPI_NONE = 0,
  ZK_EPI_BIAS = 1,
  ZK_EPI_BIAS_GELU_ERF = 2,
  ZK_EPI_BIAS_GELU_TANH = 3,
  ZK_EPI_BIAS_RESIDUAL = 4,
  ZK_EPI_BIAS_RELU = 5
} zk_epilogue;

/* Library information. */
const char *zk_last_error(void);
int zk_version(void);

/* Measurement aid, no counterpart in the reference: the shader clock under
 * sustained matrix-core load, with which the benchmark confirms the peak its
 * roofline fractions divide by. `grid` workgroups of eight wavefronts each
 * run 4 x n_mfma independent 32x32x16 fp16 MFMAs; out (device, int64
 * [grid][2]) receives each workgroup's shader-clock cycles and wall-clock
 * ticks, khz (host, int64 [2]) the wall clock's rate and the device's
 * maximum shader clock, in kHz. */
int zk_clock_probe(int grid, int n_mfma, int64_t *out, int64_t *khz, void *stream);

/* y = max(x, 0), n elements, dtype ZK_F32 or ZK_F16. x may equal y.
 * Replaces zenith_cuda.relu: core/bindings/cuda_bindings.cpp:39-46 ->
 * relu_f32 core/src/cuda_kernels.cu:504-507. */
int zk_relu(const void *x, void *y, int64_t n, int dtype, void *stream);

/* y = 1 / (1 + exp(-x)), n elements, dtype ZK_F32 or ZK_F16. x may equal y.
 * The kernel behind the ONNX Sigmoid operator's GPU branch
 * (zenith/execution/operators/activation_ops.py:82-91, which calls
 * _zenith_core.cuda.sigmoid_gpu; the reference binds no such function, so
 * its branch always falls back to NumPy). */
int zk_sigmoid(const void *x, void *y, int64_t n, int dtype, void *stream);

/* y = tanh(x), n elements, dtype ZK_F32 or ZK_F16. x may equal y. The
 * kernel behind the ONNX Tanh operator's GPU branch (activation_ops.py:111-120,
 * cuda.tanh_gpu, likewise unbound in the reference) and the BERT pooler. */
int zk_tanh(const void *x, void *y, int64_t n, int dtype, void *stream);

/* y[r, c] = GELU(x[r, c] + bias[c]); bias may be NULL. rows*cols elements,
 * contiguous. dtype ZK_F32 or ZK_F16 (fp32 math either way).
 * Replaces zenith_cuda.gelu (cuda_bindings.cpp:48-56 -> cuda_kernels.cu:
 * 115-126, 559-562) and the bias+GELU epilogue fused_bias_gelu
 * (core/src/fused_kernels.cu:47-62, 347-353). */
int zk_gelu(const void *x, const void *bias, void *y, int64_t rows,
            int64_t cols, int mode, int dtype, void *stream);

/* y = LayerNorm(x [+ residual]) * gamma + beta over the last dim (hidden),
 * population variance, fp32 statistics. residual may be NULL; x, residual, y
 * are [rows, hidden] contiguous in dtype; gamma/beta are [hidden] in dtype.
 * Replaces zenith_cuda.layernorm (cuda_bindings.cpp:58-71 ->
 * cuda_kernels.cu:132-184, 564-575) and fused_add_layernorm
 * (fused_kernels.cu:145-221, 393-399; CPU form
 * python/src/features_bindings.hpp:116-171). */
int zk_layernorm(const void *x, const void *residual, const void *gamma,
                 const void *beta, void *y, int64_t rows, int64_t hidden,
                 float eps, int dtype, void *stream);

/* y = LayerNorm(x) * gamma + beta + residual (the residual is added AFTER
 * normalisation), same shapes, dtypes and statistics as zk_layernorm;
 * residual must not be NULL. Replaces fused_layernorm_add
 * (core/src/fused_kernels.cu:224-296, 401-407), the kernel of the GraphIR
 * `LayerNormAdd` node that FusionPass emits for LayerNormalization -> Add
 * (zenith/optimization/fusion_pass.py:295-303). The reference's single-pass
 * variance E[x^2] - mean^2 (fused_kernels.cu:242-283) is replaced by exact
 * two-pass statistics. */
int zk_layernorm_add(const void *x, const void *residual, const void *gamma,
                     const void *beta, void *y, int64_t rows, int64_t hidden,
                     float eps, int dtype, void *stream);

/* zk_layernorm (fp16) that also writes q = quant(y, q_scale) as int8
 * [rows, hidden] (quant as in zk_quantize_i8, applied to the fp16 output),
 * for an int8 GEMM that consumes the normalised rows. Equals zk_layernorm
 * followed by zk_quantize_i8 on y: fused_add_layernorm
 * (fused_kernels.cu:145-221) followed by quantize_f32_to_int8_kernel
 * (cuda_kernels.cu:918-937). */
int zk_layernorm_q8(const void *x, const void *residual, const void *gamma,
                    const void *beta, void *y, int8_t *q, int64_t rows,
                    int64_t hidden, float eps, float q_scale, void *stream);

/* zk_layernorm_q8 whose residual is itself the LayerNorm of the given rows:
 *   y = LN(x + LN'(residual); gamma, beta),  q = quant(y, q_scale)
 *   LN'(r)[i, j] = (r[i, j] - mean_i) rstd_i res_gamma[j] + res_beta[j]
 * with (mean_i, rstd_i) = res_ln [rows][2] (fp32, 8-byte aligned, as the
 * LayerNorm-folded GEMMs write them), computed in fp32 without rounding
 * LN'(r) to fp16. fp16 x, residual, gammas, betas and y. No single
 * reference counterpart: the previous layer's closing Add+LayerNorm
 * (layernorm_fp16_gpu, benchmarks/bert_fp16_full.py:141-143) left
 * unmaterialised and applied where its output is the residual of this
 * layer's Add+LayerNorm (:128-130, fused_add_layernorm
 * fused_kernels.cu:145-221), followed by the int8 quantisation of the INT8
 * FFN input (quantize_f32_to_int8_kernel cuda_kernels.cu:918-937). */
int zk_layernorm_q8_res_ln(const void *x, const void *residual, const float *res_ln,
                           const void *res_gamma, const void *res_beta, const void *gamma,
                           const void *beta, void *y, int8_t *q, int64_t rows, int64_t hidden,
                           float eps, float q_scale, void *stream);

/* Out-of-place transpose of a [rows, cols] fp16 matrix (leading dim lds)
 * into [cols, rows] (leading dim ldd). Used to present B[K,N] as the
 * K-major operand the MFMA GEMM reads.
 * Replaces the layout shuffles transpose_0213 (cuda_kernels.cu:623-678). */
int zk_transpose_f16(const void *src, void *dst, int64_t rows, int64_t cols,
                     int64_t lds, int64_t ldd, void *stream);

/* FP16 GEMM on MFMA, fp32 accumulation:
 *   C[M,N] = epilogue(A[M,K] . op(B))
 *   trans_b = 1: B is W[N,K] (torch Linear layout), op(B) = W^T;
 *   trans_b = 0: B is [K,N] row-major (wmma_matmul layout).
 * out_dtype ZK_F32 or ZK_F16; bias/residual as in zk_epilogue (may be NULL
 * for ZK_EPI_NONE). A, B, C must not alias.
 * Replaces zenith_cuda.wmma_matmul (cuda_bindings.cpp:110-132 ->
 * cuda_kernels.cu:698-767) and the Linear+GELU epilogue
 * fused_gemm_epilogue_gelu (fused_kernels.cu:317-330, 416-420). */
int zk_gemm_f16(const void *A, const void *B, void *C, int64_t M, int64_t N,
                int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int trans_b,
                int out_dtype, const void *bias, const void *residual,
                int64_t ldr, int epilogue, void *stream);

/* FP32 GEMM, C[M,N] = A[M,K] . op(B), trans_b as above, fp32 throughout
 * (with trans_b and 16-byte aligned rows, K % 4 == 0: fp32 MFMA products
 * with fp32 accumulation; otherwise the SIMT kernel).
 * Replaces zenith_cuda.matmul (cuda_bindings.cpp:73-88 ->
 * matmul_f32 cuda_kernels.cu:297-336, 524-528). */
int zk_gemm_f32(const float *A, const float *B, float *C, int64_t M,
                int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                int trans_b, void *stream);

/* Fused QKV projection + attention for sequences of 64 or 128 tokens and
 * head_dim 64, fp16:
 *   qkv = X[B*S, H] . Wqkv^T + bqkv   (Wqkv [3H, H] with the rows of each
 *                                      head interleaved: q_h, k_h, v_h,
 *                                      64 rows each, h = 0 .. heads-1)
 *   ctx[b*S + s, 64h .. 64h+63] = softmax(scale * q . k^T) . v per (b, h),
 *                                 keys j >= valid_lens[b] masked as in
 *                                 zk_flash_attn_fwd (valid_lens may be NULL)
 * Q, K and V stay on chip: each 256-row x 192-column GEMM tile holds one
 * head of 256 / S whole sequences and runs their attention in its epilogue.
 * The values equal the unfused pair zk_gemm_f16 (bias epilogue, fp16 out)
 * + zk_flash_attn_fwd to fp16 rounding of the attention output. H must be
 * heads * 64; X and Wqkv 16-byte aligned, ctx 8-byte aligned, rows dense.
 * No single reference counterpart: replaces the QKV linear_fp16_gpu calls,
 * the transposes and attention_full_fp16_gpu of the reference encoder layer
 * (benchmarks/bert_fp16_full.py:98-121), i.e. zenith_cuda.wmma_matmul and
 * zenith_cuda.flash_attention (cuda_bindings.cpp:90-132). */
int zk_qkv_attn_f16(const void *X, const void *Wqkv, const void *bqkv, void *ctx,
                    int64_t batch, int64_t seq, int64_t hidden, int64_t heads,
                    const int32_t *valid_lens, float scale, void *stream);

/* The same with the LayerNorm of X's rows folded in: X holds the LN input
 * x, Wqkv is gamma-scaled (W'[n,k] = W[n,k] gamma[k], rows interleaved per
 * head as above), and q, k, v = rstd (x . W'^T - mean ln_s) + ln_c with
 * ln_s[n] = sum_k W'[n,k] and ln_c = beta . W^T + bias (fp32 [3H], 16-byte
 * aligned). The row statistics come from ln_part [B*S][H/96][2]: (mean, M2)
 * of every 96-column segment of the row (as zk_gemm_f16_res_stats writes
 * them), merged in a fixed order; (mean, rstd) of every row go to ln_out
 * [B*S][2] when it is not NULL. H a multiple of 96, at most 1536;
 * statistics arrays 8-byte aligned. No reference counterpart: the LayerNorm
 * before the QKV projection (the previous reference layer's final one,
 * benchmarks/bert_fp16_full.py:142-143, layernorm_fp16_gpu) folded into it. */
int zk_qkv_attn_f16_ln(const void *X, const void *Wqkv, const float *ln_part, float ln_eps,
                       const float *ln_s, const float *ln_c, float *ln_out, void *ctx,
                       int64_t batch, int64_t seq, int64_t hidden, int64_t heads,
                       const int32_t *valid_lens, float scale, void *stream);

/* zk_qkv_attn_f16 (ln_part NULL, bqkv used) or zk_qkv_attn_f16_ln (ln_part
 * set, bqkv ignored) with ctx written in fragment order (defined below, at
 * zk_gemm_f16_ln_frag: ceil(B*S/32) * 32 x hidden halves, rows past B*S not
 * written, 16-byte aligned), the A operand of zk_gemm_f16_res_stats_frag for
 * the out-projection. The values are those entry points', bit for bit. No
 * reference counterpart (the layout of the attention output the reference
 * hands to its out-projection, benchmarks/bert_fp16_full.py:118-126). */
int zk_qkv_attn_f16_frag(const void *X, const void *Wqkv, const void *bqkv, const float *ln_part,
                         float ln_eps, const float *ln_s, const float *ln_c, float *ln_out,
                         void *ctx, int64_t batch, int64_t seq, int64_t hidden, int64_t heads,
                         const int32_t *valid_lens, float scale, void *stream);

/* fp16 GEMM with a residual and the row statistics of its output:
 *   C = A[M,K] . W[N,K]^T + bias + R,  R = res, or with res_ln [M][2]
 *       (mean, rstd per row): R = (res - mean) rstd gamma + beta
 *   part_out [M][N/96][2] = (mean, M2) of each 96-column segment of each
 *       row of C as stored (fp16-rounded values)
 * N a multiple of 96; K, lda, ldw, ldc, ldr multiples of 8; A, W, C, res,
 * gamma, beta 16-byte aligned; res_ln and part_out 8-byte aligned. With
 * res_ln it is the reference's residual add of a LayerNorm output
 * (benchmarks/bert_fp16_full.py:128-130, 141-143: add_fp16_gpu of the
 * previous layernorm_fp16_gpu result) with that LayerNorm computed on the
 * fly; the statistics let the next GEMM fold the following LayerNorm
 * (zk_gemm_f16_ln). No single reference counterpart. */
int zk_gemm_f16_res_stats(const void *A, const void *W, void *C, int64_t M, int64_t N,
                          int64_t K, int64_t lda, int64_t ldw, int64_t ldc,
                          const void *bias, const void *res, int64_t ldr, const float *res_ln,
                          const void *res_gamma, const void *res_beta, float *part_out,
                          void *stream);

/* fp16 GEMM on LayerNorm-ed rows, the LayerNorm folded into the weights:
 *   C = act(rstd (A . W'^T - mean ln_s) + ln_c)
 * A holds the LN input; W' = gamma-scaled weights (W'[n,k] = W[n,k]
 * gamma[k]), ln_s[n] = sum_k W'[n,k], ln_c = beta . W^T + bias (fp32 [N],
 * 16-byte aligned); per-row statistics from ln_part [M][K/96][2] as for
 * zk_qkv_attn_f16_ln, (mean, rstd) written to ln_out [M][2] if not NULL.
 * K a multiple of 96, at most 1536; epilogue ZK_EPI_BIAS (no activation) or
 * ZK_EPI_BIAS_GELU_ERF. Replaces layernorm_fp16_gpu + linear_fp16_gpu +
 * gelu_fp16_gpu of the reference layer (benchmarks/bert_fp16_full.py:
 * 129-134). */
int zk_gemm_f16_ln(const void *A, const void *W, void *C, int64_t M, int64_t N, int64_t K,
                   int64_t lda, int64_t ldw, int64_t ldc, const float *ln_part, float ln_eps,
                   const float *ln_s, const float *ln_c, float *ln_out, int epilogue,
                   void *stream);

/* Fragment order: the layout of an fp16 matrix X [R][K] (K a multiple of 16)
 * in which it feeds a 32x32x16 MFMA as the A operand straight from memory.
 * For row block rb (rows 32 rb .. 32 rb + 31) and k-step ks (columns
 * 16 ks .. 16 ks + 15), the 512 halves at element (rb * K / 16 + ks) * 512
 * hold, for lane l = 0 .. 63, X[32 rb + l % 32][16 ks + 8 (l / 32) + e] at
 * element 8 l + e (e = 0 .. 7). A fragment-ordered buffer holds whole row
 * blocks: ceil(R / 32) * 32 rows.
 *
 * zk_gemm_f16_ln with ZK_EPI_BIAS_GELU_ERF, C written in fragment order
 * (ceil(M/32) * 32 x N; rows past M are not written). N a multiple of 64.
 * The values are zk_gemm_f16_ln's, bit for bit. No reference counterpart:
 * the FFN intermediate between the two FFN GEMMs of the reference layer
 * (benchmarks/bert_fp16_full.py:133-139) laid out for zk_gemm_f16_res_stats_frag. */
int zk_gemm_f16_ln_frag(const void *A, const void *W, void *C, int64_t M, int64_t N, int64_t K,
                        int64_t lda, int64_t ldw, const float *ln_part, float ln_eps,
                        const float *ln_s, const float *ln_c, float *ln_out, void *stream);

/* zk_gemm_f16_res_stats with A in fragment order (ceil(M/32) * 32 x K; rows
 * past M are read and their products discarded). K a multiple of 64. Each
 * 1 KB fragment reaches LDS with one contiguous DMA instruction and is read
 * back linearly. Runs the 128x96 tile at every M; the values and statistics
 * are zk_gemm_f16_res_stats's, bit for bit, wherever that takes the same
 * tile (M < 10240 at N = 768). No reference counterpart (see
 * zk_gemm_f16_ln_frag). */
/* C[M,N] = A . W^T + bias, fp16 out (row-major), A in fragment order
 * (ceil(M/32) * 32 x K; rows past M read and discarded; K a multiple of 64):
 * the INT8-FFN layer's out-projection on the fused attention's output. The
 * 128x96 tile at every M. No reference counterpart (the out-projection
 * linear_fp16_gpu, benchmarks/bert_fp16_full.py:124-126, on this layout). */
int zk_gemm_f16_frag(const void *A, const void *W, void *C, int64_t M, int64_t N, int64_t K,
                     int64_t ldw, int64_t ldc, const void *bias, void *stream);

int zk_gemm_f16_res_stats_frag(const void *A, const void *W, void *C, int64_t M, int64_t N,
                               int64_t K, int64_t ldw, int64_t ldc, const void *bias,
                               const void *res, int64_t ldr, const float *res_ln,
                               const void *res_gamma, const void *res_beta, float *part_out,
                               void *stream);

/* Flash-attention forward, non-causal, online softmax with fp32 statistics.
 *   O[b,h,s,:] = softmax(scale * Q[b,h,s,:] . K[b,h,:,:]^T) . V[b,h,:,:]
 * Tensors are addressed by strides (elements): strides[0..2] are the
 * (batch, head, seq) strides of Q, [3..5] of K, [6..8] of V, [9..11] of O;
 * the head_dim axis is contiguous. Any head_dim <= 128 (the reference's
 * HEAD_DIM_MAX, flash_attention.cu:26); fp16 needs a multiple of 8. Kernels
 * are compiled for widths 32, 64 and 128; other widths are zero-padded
 * inside the kernel.
 * valid_lens (int32 [B], may be NULL): keys j >= valid_lens[b] are masked
 * (probability exactly 0); a row with no valid key yields 0.
 * dtype ZK_F16 (MFMA path) or ZK_F32 (fp32 path).
 * Replaces zenith_cuda.flash_attention (cuda_bindings.cpp:90-106 ->
 * flash_attention_forward core/src/flash_attention.cu:194-340) and its
 * unbound FP16 twin (flash_attention.cu:55-188); mask rule from
 * zenith/jax/primitives.py:302-310. */
int zk_flash_attn_fwd(const void *Q, const void *K, const void *V, void *O,
                      int64_t batch, int64_t heads, int64_t seq_q,
                      int64_t seq_k, int64_t head_dim, const int64_t *strides,
                      const int32_t *valid_lens, float scale, int dtype,
                      void *stream);

/* zk_flash_attn_fwd with a boolean attention mask on top of valid_lens
 * (which may be NULL): mask[b, h, q, k] != 0 keeps key k for query q, 0
 * gives it probability exactly 0; a query with no kept key yields 0.
 * mask is uint8, one byte per key with keys contiguous; mask_strides[0..2]
 * are its (batch, head, query) strides in bytes, multiples of 4 (0
 * broadcasts), mask is 4-byte aligned, and every row holds seq_k rounded up
 * to a multiple of 4 bytes (keys are read 4 at a time; bytes past seq_k are
 * ignored). This is the boolean attn_mask of
 * scaled_dot_product_attention, [B|1, H|1, Sq|1, Sk], which the reference's
 * FX replacement hands to torch (zenith/optimization/fx_patterns.py:106-114),
 * with the masked-attention rule of zenith/jax/primitives.py:302-310. */
int zk_flash_attn_fwd_masked(const void *Q, const void *K, const void *V, void *O,
                             int64_t batch, int64_t heads, int64_t seq_q, int64_t seq_k,
                             int64_t head_dim, const int64_t *strides,
                             const int32_t *valid_lens, const uint8_t *mask,
                             const int64_t *mask_strides, float scale, int dtype,
                             void *stream);

/* Symmetric int8 quantisation, q = clamp(round_half_even(x / scale),
 * -128, 127), x in dtype ZK_F32 or ZK_F16 (n elements, contiguous).
 * Replaces quantize_f32_to_int8_kernel (cuda_kernels.cu:918-937; numpy form
 * benchmarks/int8_bench.py:19-27). */
int zk_quantize_i8(const void *x, int8_t *q, int64_t n, float scale,
                   int dtype, void *stream);

/* INT8 GEMM on MFMA with int32 accumulation:
 *   acc[M,N] = A_q[M,K] . W_q[N,K]^T   (both int8, K-major)
 *   out_dtype ZK_I32: C = acc (raw accumulators; epilogue must be NONE)
 *   out_dtype ZK_F16 / ZK_F32: C = epilogue(acc * (s_x * s_w[n]))
 * s_w is fp32 [N] (per-output-channel weight scales), s_x the per-tensor
 * activation scale; bias/residual in out_dtype.
 * Replaces int8_matmul / fused_int8_linear (cuda_kernels.cu:963-1049;
 * numpy form benchmarks/int8_bench.py:42-45). */
int zk_gemm_i8(const int8_t *A, const int8_t *W, void *C, int64_t M,
               int64_t N, int64_t K, int64_t lda, int64_t ldw, int64_t ldc,
               float s_x, const float *s_w, const void *bias,
               const void *residual, int64_t ldr, int epilogue,
               int out_dtype, void *stream);

/* INT8 GEMM whose output is re-quantised for the next int8 GEMM:
 *   Q[m,n] = quant(fp16(epilogue(acc[m,n] * (s_x * s_w[n]) + bias[n])), s_out)
 * with quant as in zk_quantize_i8; bias fp16 [N]; epilogue NONE, BIAS,
 * BIAS_GELU_ERF, BIAS_GELU_TANH or BIAS_RELU. Q is int8 [M, ldq].
 * Equals zk_gemm_i8 (out_dtype ZK_F16) followed by zk_quantize_i8 on its
 * output, without the fp16 intermediate: the FFN-up -> quantise step of the
 * INT8 FFN (fused_int8_linear cuda_kernels.cu:1010-1049 followed by
 * quantize_f32_to_int8_kernel :918-937; numpy form
 * benchmarks/int8_bench.py:19-45). */
int zk_gemm_i8_requant(const int8_t *A, const int8_t *W, int8_t *Q, int64_t M,
                       int64_t N, int64_t K, int64_t lda, int64_t ldw, int64_t ldq,
                       float s_x, const float *s_w, const void *bias, int epilogue,
                       float s_out, void *stream);

/* zk_gemm_f16_res_stats on the int8 product, dequantised as in zk_gemm_i8:
 *   C = acc[m,n] * (s_x * s_w[n]) + bias[n] + R,  R = res, or with res_ln
 *       its LayerNorm as in zk_gemm_f16_res_stats
 *   part_out [M][N/96][2] = (mean, M2) of each 96-column segment of each row
 *       of C as stored (fp16)
 * fp16 C, bias, res (and res_gamma, res_beta); operand rules of zk_gemm_i8,
 * N a multiple of 96, ldc and ldr multiples of 8, C and res 16-byte aligned.
 * No single reference counterpart: the INT8 FFN-down (fused_int8_linear
 * cuda_kernels.cu:1010-1049) with the residual add of the layer's closing
 * Add+LayerNorm (benchmarks/bert_fp16_full.py:141-143) and the statistics
 * that let the next layer fold that LayerNorm in. */
int zk_gemm_i8_res_stats(const int8_t *A, const int8_t *W, void *C, int64_t M, int64_t N,
                         int64_t K, int64_t lda, int64_t ldw, int64_t ldc, float s_x,
                         const float *s_w, const void *bias, const void *res, int64_t ldr,
                         const float *res_ln, const void *res_gamma, const void *res_beta,
                         float *part_out, void *stream);

/* The INT8 FFN's intermediate in fragment order: the fp16 definition above
 * with 32 int8 columns per k-step (lane l holds X[32 rb + l % 32][32 ks +
 * 16 (l / 32) + e] at byte 16 l + e, e = 0 .. 15), the A operand of a
 * 32x32x32 int8 MFMA. zk_gemm_i8_requant_frag writes zk_gemm_i8_requant's
 * values (bit for bit) that way (ceil(M/32) * 32 x N bytes, rows past M not
 * written; N a multiple of 128, Q 16-byte aligned); zk_gemm_i8_res_stats_frag
 * is zk_gemm_i8_res_stats on such an A (K a multiple of 128; rows past M read
 * and discarded; the 128x96 tile at every M, bit for bit with
 * zk_gemm_i8_res_stats wherever that takes the same tile). No reference
 * counterpart: the int8 intermediate between the reference's INT8 FFN
 * linears (benchmarks/int8_bench.py:19-45) laid out for the second one. */
int zk_gemm_i8_requant_frag(const int8_t *A, const int8_t *W, int8_t *Q, int64_t M, int64_t N,
                            int64_t K, int64_t lda, int64_t ldw, float s_x, const float *s_w,
                            const void *bias, int epilogue, float s_out, void *stream);
int zk_gemm_i8_res_stats_frag(const int8_t *A, const int8_t *W, void *C, int64_t M, int64_t N,
                              int64_t K, int64_t ldw, int64_t ldc, float s_x, const float *s_w,
                              const void *bias, const void *res, int64_t ldr,
                              const float *res_ln, const void *res_gamma, const void *res_beta,
                              float *part_out, void *stream);

/* c[r, :] = a[r, :] + b[b_rows == 1 ? 0 : r, :] for [rows, cols] contiguous
 * tensors in dtype ZK_F32 or ZK_F16 (fp16 summed in fp32, rounded once);
 * b_rows is 1 (row broadcast: bias) or rows.
 * Replaces add_2d_f32 and add_bias_f32 (core/src/cuda_kernels.cu:582-616)
 * and add_fp16 (core/src/fp16_kernels.cu:267-280). */
int zk_add(const void *a, const void *b, void *c, int64_t rows, int64_t cols,
           int64_t b_rows, int dtype, void *stream);

/* Row softmax y = exp(x - max) / sum over the last dim of [rows, cols]
 * contiguous, fp32 math (exact expf), dtype ZK_F32 or ZK_F16.
 * Replaces softmax_2d_f32 (core/src/cuda_kernels.cu:220-246, 577-580; CPU
 * form softmax_f32, core/src/cpu_kernels.cpp:382-408). */
int zk_softmax(const void *x, void *y, int64_t rows, int64_t cols, int dtype,
               void *stream);

/* y[i][k][j][l] = x[i][j][k][l] for contiguous x of shape [d0, d1, d2, d3]
 * (attention head split / merge: [B,S,H,D] <-> [B,H,S,D]), dtype ZK_F32
 * or ZK_F16, not in place.
 * Replaces transpose_0213_f32 / transpose_0213_inv_f32
 * (core/src/cuda_kernels.cu:623-678) and their fp16 twins
 * (core/src/fp16_kernels.cu:285-325). */
int zk_transpose_0213(const void *x, void *y, int64_t d0, int64_t d1, int64_t d2,
                      int64_t d3, int dtype, void *stream);

/* n-element conversion between ZK_F32 and ZK_F16 (round to nearest even).
 * Replaces convert_f32_to_f16 / convert_f16_to_f32
 * (core/src/fp16_kernels.cu:50-77) and convert_fp32_to_fp16 (fp16_ops.cu:56). */
int zk_convert(const void *x, void *y, int64_t n, int src_dtype, int dst_dtype,
               void *stream);

/* Workspace for the split-K form of the GEMMs: bytes zk_gemm_f16_ws /
 * zk_gemm_f32_ws (dtype ZK_F16 / ZK_F32) use for an M x N x K product, 0 when
 * the product is not split. Small-M products (too few 64x64 tiles to fill
 * the GPU) are split along K; each split writes an fp32 partial tile to the
 * workspace and a reduction sums the splits in order (deterministic) and
 * applies the epilogue. The workspace is the caller's (the library
 * allocates nothing); no counterpart in the reference, whose
 * cuBLAS calls hid their own workspaces (python/src/bindings.cpp:1454-1498). */
int64_t zk_gemm_workspace_size(int64_t M, int64_t N, int64_t K, int dtype);

/* zk_gemm_f16 with a caller workspace of ws_bytes (see
 * zk_gemm_workspace_size); with a null or too small workspace it is
 * zk_gemm_f16. */
int zk_gemm_f16_ws(const void *A, const void *B, void *C, int64_t M, int64_t N,
                   int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int trans_b,
                   int out_dtype, const void *bias, const void *residual, int64_t ldr,
                   int epilogue, void *workspace, int64_t ws_bytes, void *stream);

/* Linear + residual + LayerNorm (the post-LN block closing a BERT attention
 * or FFN half), fp16:
 *   T = fp16(A[M,K] . W[N,K]^T + bias),  Y = LayerNorm(T + R) * gamma + beta
 * bit-identical to zk_gemm_f16_ws (ZK_EPI_BIAS, fp16 out, ldc = N) into T
 * followed by zk_layernorm(T, R). When the product splits along K (a
 * workspace of at least zk_gemm_workspace_size(M, N, K, ZK_F16) bytes, as
 * for zk_gemm_f16_ws), N is a multiple of 8 with 16-byte aligned bias, R,
 * gamma, beta and Y, and either M < 2048 with N <= 1024 or at most M / 32
 * splits with N <= 8192, the split partials are read straight by the
 * LayerNorm launch, which forms the rows of T itself: one launch fewer, and
 * T is not written. Otherwise T ([M, N] fp16, contiguous) holds the product
 * as the pair would leave it. R, Y: [M, N] contiguous; bias,
 * gamma, beta: [N]. Operand rules of zk_gemm_f16 (W as [N, K], K, lda, ldw
 * multiples of 8, A and W 16-byte aligned). No single reference
 * counterpart: the out-projection / FFN-down linear and the Add+LayerNorm
 * after it (benchmarks/bert_fp16_full.py:128-143; fused_add_layernorm
 * core/src/fused_kernels.cu:145-221). */
int zk_gemm_f16_add_ln(const void *A, const void *W, const void *bias, const void *R,
                       const void *gamma, const void *beta, void *T, void *Y, int64_t M,
                       int64_t N, int64_t K, int64_t lda, int64_t ldw, float eps,
                       void *workspace, int64_t ws_bytes, void *stream);

/* zk_gemm_f16 that allocates nothing and takes no workspace: for callers
 * that cannot allocate device memory (code under HIP-graph capture, tight
 * serving loops, hosts that forbid allocation). No counterpart in the
 * reference. Same arguments, checks and results as zk_gemm_f16_ws with a
 * workspace of zk_gemm_workspace_size(M, N, K, ZK_F16) bytes: small-M
 * products are split along K, their fp32 partials kept in a static 8 MiB
 * device array (one per GPU, held until the process ends; the split plan
 * never needs more, and a larger need is rejected with ZK_ERR_UNSUPPORTED).
 * The first call on each device that splits looks up the array's address on
 * that device (hipGetSymbolAddress) and must run outside graph capture; later
 * calls make no HIP call besides their launches and can be captured.
 * Calls that overlap in time on one GPU race on that array. */
int zk_gemm_f16_noalloc(const void *A, const void *B, void *C, int64_t M, int64_t N,
                        int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int trans_b,
                        int out_dtype, const void *bias, const void *residual, int64_t ldr,
                        int epilogue, void *stream);

/* zk_gemm_f32 with a caller workspace of ws_bytes (split-K on the fp32
 * MFMA path); with a null or too small workspace it is zk_gemm_f32. */
int zk_gemm_f32_ws(const float *A, const float *B, float *C, int64_t M, int64_t N,
                   int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int trans_b,
                   void *workspace, int64_t ws_bytes, void *stream);

/* Y[M,N] = epilogue(X[M,K] . W[N,K]^T) in fp32 (torch Linear layout), with
 * the epilogues of zk_gemm_f16 (bias, bias+GELU erf / tanh, bias+residual,
 * bias+ReLU; `bias` fp32 [N], `residual` fp32 [M, ldr]) fused into the GEMM
 * (or into its split-K reduction) and an optional caller workspace as for
 * zk_gemm_f32_ws. Replaces the fp32 linear of the GPU tensor API,
 * linear_gpu (python/src/bindings.cpp:1454-1498: cuBLAS SGEMM, then a bias
 * kernel) and zenith_cuda's fp32 Linear (cuda_bindings.cpp:73 matmul, then
 * bias and activation kernels). */
int zk_linear_f32(const float *X, const float *W, float *Y, int64_t M, int64_t N, int64_t K,
                  int64_t ldx, int64_t ldw, int64_t ldy, const float *bias,
                  const float *residual, int64_t ldr, int epilogue, void *workspace,
                  int64_t ws_bytes, void *stream);

/* Embedding gather, out[i, :] = table[ids[i], :] for int32 ids [n] and a
 * [vocab, hidden] table in dtype ZK_F32 or ZK_F16; an id outside [0, vocab)
 * gives a zero row. Replaces embedding_f32
 * (core/src/transformer_kernels.cu:236-262). */
int zk_embedding(const int32_t *ids, const void *table, void *out, int64_t n,
                 int64_t hidden, int64_t vocab, int dtype, void *stream);

/* BERT input layer in one pass per token:
 *   out[b, s, :] = LayerNorm(word[ids[b,s]] + pos[s + pos_offset]
 *                            + type[token_type_ids[b,s]]) * gamma + beta
 * ids / token_type_ids int32 [batch, seq] (token_type_ids may be NULL: type
 * 0); tables [vocab | max_pos | n_types, hidden] and gamma / beta [hidden] in
 * dtype ZK_F32 or ZK_F16; fp32 two-pass statistics; hidden a multiple of the
 * 16-byte vector and at most 4096 (fp16) / 2048 (fp32). An id outside its
 * table contributes nothing. The composition of the reference's embedding
 * gather (transformer_kernels.cu:236-262) with the HF BertEmbeddings sum and
 * LayerNorm that its loaders target (benchmarks/bert_fp16_full.py:45-94). */
int zk_bert_embeddings(const int32_t *input_ids, const int32_t *token_type_ids,
                       const void *word, const void *pos, const void *type_table,
                       const void *gamma, const void *beta, void *out, int64_t batch,
                       int64_t seq, int64_t hidden, int64_t vocab, int64_t max_pos,
                       int64_t n_types, int64_t pos_offset, float eps, int dtype,
                       void *stream);

#ifdef __cplusplus
}
#endif

#endif /* ZK_API_H */

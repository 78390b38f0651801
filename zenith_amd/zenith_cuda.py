"""`zenith_cuda` drop-in: the reference's native kernel module on MI355X.

Same entry points, positional signatures, output dtypes/shapes and
RuntimeError preconditions as the reference torch extension
(core/bindings/cuda_bindings.cpp:39-145):

    relu(input)                                  cuda_bindings.cpp:39-46
    gelu(input)                                  cuda_bindings.cpp:48-56 (tanh GELU)
    layernorm(input, gamma, beta, eps=1e-5)      cuda_bindings.cpp:58-71, 139-140
    matmul(A, B)                                 cuda_bindings.cpp:73-88 (fp32)
    flash_attention(Q, K, V)                     cuda_bindings.cpp:90-106
    wmma_matmul(A, B)                            cuda_bindings.cpp:110-132 (f16 in, f32 out)

Differences that only add behaviour: fp16 inputs are accepted where the
reference is fp32-only, `wmma_matmul` takes `out_dtype`, `flash_attention`
takes `key_padding_lengths` / `scale`, and the fused entry points used by the
graph hooks are exported (`add_layernorm`, `bias_gelu`, `linear`,
`quantize_int8`, `int8_linear`, `int8_matmul`).

Every call launches on torch's current stream of the input's device (the
reference used the legacy default stream) and allocates its outputs with the
torch caching allocator; nothing synchronises.
"""

from __future__ import annotations

import math

import torch

from . import _lib as L

_DT = {torch.float32: L.ZK_F32, torch.float16: L.ZK_F16}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _p(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _need_cuda(*ts, msg="Input must be CUDA tensor"):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError(msg)
    dev = None
    for t in ts:
        if t is None:
            continue
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError("All tensors must be on the same device")


def _float_dtype(t: torch.Tensor, who: str) -> int:
    if t.dtype not in _DT:
        raise RuntimeError(f"{who}: expected float32 or float16, got {t.dtype}")
    return _DT[t.dtype]


# --------------------------------------------------------------- activations
def relu(input: torch.Tensor) -> torch.Tensor:
    """ReLU on a new tensor (reference clones then applies in place)."""
    _need_cuda(input)
    if not input.is_contiguous():
        raise RuntimeError("Input must be contiguous")
    dt = _float_dtype(input, "relu")
    out = torch.empty_like(input)
    L.call("zk_relu", _p(input), _p(out), input.numel(), dt, _stream(input))
    return out


def gelu(input: torch.Tensor, approximate: str = "tanh") -> torch.Tensor:
    """GELU; the reference kernel is the tanh approximation (the default)."""
    return bias_gelu(input, None, approximate=approximate)


def bias_gelu(input: torch.Tensor, bias: torch.Tensor | None,
              approximate: str = "tanh") -> torch.Tensor:
    """GELU(input + bias[col]) over the last dimension (fused_bias_gelu,
    core/src/fused_kernels.cu:47-62)."""
    _need_cuda(input, bias)
    if not input.is_contiguous():
        raise RuntimeError("Input must be contiguous")
    dt = _float_dtype(input, "gelu")
    mode = {"tanh": L.ZK_GELU_TANH, "none": L.ZK_GELU_ERF, "erf": L.ZK_GELU_ERF}.get(approximate)
    if mode is None:
        raise RuntimeError(f"gelu: approximate must be 'tanh' or 'none', got {approximate!r}")
    cols = input.shape[-1] if input.dim() > 0 else 1
    rows = input.numel() // cols if cols else 0
    if bias is not None:
        if bias.dtype != input.dtype or bias.numel() != cols:
            raise RuntimeError("bias must match the input dtype and last dimension")
        bias = bias.contiguous()
    out = torch.empty_like(input)
    L.call("zk_gelu", _p(input), _p(bias), _p(out), rows, cols, mode, dt, _stream(input))
    return out


# ------------------------------------------------------------------- norms --
def layernorm(input: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor,
              eps: float = 1e-5) -> torch.Tensor:
    """LayerNorm over the last dim of a 2-D [batch, hidden] tensor."""
    return add_layernorm(input, None, gamma, beta, eps)


def add_layernorm(input: torch.Tensor, residual: torch.Tensor | None,
                  gamma: torch.Tensor, beta: torch.Tensor,
                  eps: float = 1e-5) -> torch.Tensor:
    """LayerNorm(input + residual) (fused_add_layernorm,
    core/src/fused_kernels.cu:145-221; CPU form
    python/src/features_bindings.hpp:116-171)."""
    _need_cuda(input, residual, gamma, beta)
    if input.dim() != 2:
        raise RuntimeError("Input must be 2D [batch, hidden]")
    dt = _float_dtype(input, "layernorm")
    rows, hidden = input.shape
    for t, name in ((gamma, "gamma"), (beta, "beta")):
        if t.dtype != input.dtype or t.numel() != hidden:
            raise RuntimeError(f"{name} must be [hidden] with the input dtype")
    if residual is not None and (residual.shape != input.shape or residual.dtype != input.dtype):
        raise RuntimeError("residual must match input shape and dtype")
    x = input.contiguous()
    r = residual.contiguous() if residual is not None else None
    out = torch.empty_like(x)
    L.call("zk_layernorm", _p(x), _p(r), _p(gamma.contiguous()), _p(beta.contiguous()),
           _p(out), rows, hidden, float(eps), dt, _stream(x))
    return out


def layernorm_add(input: torch.Tensor, residual: torch.Tensor, gamma: torch.Tensor,
                  beta: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """LayerNorm(input) * gamma + beta + residual, the residual added after
    normalisation (fused_layernorm_add, core/src/fused_kernels.cu:224-296,
    401-407; the kernel of the GraphIR `LayerNormAdd` node,
    zenith/optimization/fusion_pass.py:295-303)."""
    _need_cuda(input, residual, gamma, beta)
    if input.dim() != 2:
        raise RuntimeError("Input must be 2D [batch, hidden]")
    if residual is None:
        raise RuntimeError("layernorm_add needs a residual")
    dt = _float_dtype(input, "layernorm_add")
    rows, hidden = input.shape
    for t, name in ((gamma, "gamma"), (beta, "beta")):
        if t.dtype != input.dtype or t.numel() != hidden:
            raise RuntimeError(f"{name} must be [hidden] with the input dtype")
    if residual.shape != input.shape or residual.dtype != input.dtype:
        raise RuntimeError("residual must match input shape and dtype")
    x = input.contiguous()
    r = residual.contiguous()
    out = torch.empty_like(x)
    L.call("zk_layernorm_add", _p(x), _p(r), _p(gamma.contiguous()), _p(beta.contiguous()),
           _p(out), rows, hidden, float(eps), dt, _stream(x))
    return out


def add_layernorm_q8(input: torch.Tensor, residual: torch.Tensor | None,
                     gamma: torch.Tensor, beta: torch.Tensor, eps: float,
                     q_scale: float) -> tuple[torch.Tensor, torch.Tensor]:
    """fp16 LayerNorm(input + residual) and its int8 quantisation with scale
    q_scale in one pass: returns (y, quantize_int8(y, q_scale)) — the
    fused_add_layernorm -> quantize_f32_to_int8_kernel sequence
    (core/src/fused_kernels.cu:145-221, core/src/cuda_kernels.cu:918-937)."""
    _need_cuda(input, residual, gamma, beta)
    if input.dim() != 2 or input.dtype != torch.float16:
        raise RuntimeError("add_layernorm_q8: input must be 2D float16 [batch, hidden]")
    rows, hidden = input.shape
    for t, name in ((gamma, "gamma"), (beta, "beta")):
        if t.dtype != input.dtype or t.numel() != hidden:
            raise RuntimeError(f"{name} must be [hidden] with the input dtype")
    if residual is not None and (residual.shape != input.shape or residual.dtype != input.dtype):
        raise RuntimeError("residual must match input shape and dtype")
    x = input.contiguous()
    r = residual.contiguous() if residual is not None else None
    out = torch.empty_like(x)
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    L.call("zk_layernorm_q8", _p(x), _p(r), _p(gamma.contiguous()), _p(beta.contiguous()),
           _p(out), _p(q), rows, hidden, float(eps), float(q_scale), _stream(x))
    return out, q


# ------------------------------------------------------------------ GEMMs ---
def _pad_k(t: torch.Tensor, mult: int) -> torch.Tensor:
    k = t.shape[-1]
    if k % mult == 0 and t.is_contiguous() and t.data_ptr() % 16 == 0:
        return t
    kp = (k + mult - 1) // mult * mult
    out = torch.zeros(*t.shape[:-1], kp, dtype=t.dtype, device=t.device)
    out[..., :k] = t
    return out


def gemm_workspace(M: int, N: int, K: int, dtype: int, device) -> torch.Tensor | None:
    """Caller-side workspace for the split-K GEMMs (zk_gemm_workspace_size
    bytes, from torch's caching allocator), or None when the product is not
    split."""
    n = int(L.load().zk_gemm_workspace_size(M, N, K, dtype))
    return torch.empty(n, dtype=torch.uint8, device=device) if n > 0 else None


def _ws_args(ws):
    return (None, 0) if ws is None else (ws.data_ptr(), ws.numel())


def _gemm_f16_nt(a: torch.Tensor, w: torch.Tensor, out_dtype, bias=None,
                 residual=None, epilogue=L.ZK_EPI_NONE) -> torch.Tensor:
    """C[M,N] = epilogue(a[M,K] . w[N,K]^T) on the MFMA kernel (split along K
    with a workspace when M is small)."""
    M, K = a.shape
    N = w.shape[0]
    a = _pad_k(a, 8)
    w = _pad_k(w, 8)
    out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    ldr = 0
    if residual is not None:
        residual = residual.contiguous()
        ldr = residual.stride(0)
    ws = gemm_workspace(M, N, a.shape[1], L.ZK_F16, a.device) if M else None
    L.call("zk_gemm_f16_ws", _p(a), _p(w), _p(out), M, N, a.shape[1], a.stride(0),
           w.stride(0), out.stride(0), 1, _DT[out_dtype], _p(bias), _p(residual), ldr,
           epilogue, *_ws_args(ws), _stream(a))
    return out


def transpose_f16(x: torch.Tensor) -> torch.Tensor:
    """[R, C] fp16 -> contiguous [C, R] on the HIP transpose kernel."""
    _need_cuda(x)
    if x.dim() != 2 or x.dtype != torch.float16 or x.stride(1) != 1:
        raise RuntimeError("transpose_f16 expects a row-major 2-D fp16 tensor")
    R, C = x.shape
    if R > 1 and x.stride(0) < C:  # overlapping rows (e.g. a broadcast view)
        x = x.contiguous()
    out = torch.empty((C, R), dtype=torch.float16, device=x.device)
    L.call("zk_transpose_f16", _p(x), _p(out), R, C, x.stride(0) if R > 1 else C,
           out.stride(0), _stream(x))
    return out


def wmma_matmul(A: torch.Tensor, B: torch.Tensor,
                out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """C = A[M,K] . B[K,N], fp16 inputs, fp32 accumulation, fp32 output by
    default (reference semantics); out_dtype=torch.float16 for fp16 output."""
    if not (A.is_cuda and B.is_cuda):
        raise RuntimeError("Inputs must be CUDA tensors")
    _need_cuda(A, B)
    if A.dim() != 2 or B.dim() != 2:
        raise RuntimeError("Inputs must be 2D")
    if A.dtype != torch.float16:
        raise RuntimeError("A must be FP16 (use .half())")
    if B.dtype != torch.float16:
        raise RuntimeError("B must be FP16 (use .half())")
    if B.shape[0] != A.shape[1]:
        raise RuntimeError("Matrix dimensions must match")
    if out_dtype not in (torch.float32, torch.float16):
        raise RuntimeError("out_dtype must be torch.float32 or torch.float16")
    A = _rows_dense(A)
    Bc = _rows_dense(B)
    if A.shape[0] == 0 or B.shape[1] == 0:
        return torch.empty((A.shape[0], B.shape[1]), dtype=out_dtype, device=A.device)
    if A.shape[1] == 0:
        return torch.zeros((A.shape[0], B.shape[1]), dtype=out_dtype, device=A.device)
    bt = transpose_f16(Bc)  # W[N,K] view of B for the K-major MFMA kernel
    return _gemm_f16_nt(A, bt, out_dtype)


def matmul(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """C = A[M,K] . B[K,N] in fp32 (reference `matmul`). fp16 inputs are
    routed to the MFMA kernel with fp16 output."""
    if not (A.is_cuda and B.is_cuda):
        raise RuntimeError("Inputs must be CUDA tensors")
    _need_cuda(A, B)
    if A.dim() != 2 or B.dim() != 2:
        raise RuntimeError("Inputs must be 2D")
    if B.shape[0] != A.shape[1]:
        raise RuntimeError("Matrix dimensions must match")
    if A.dtype == torch.float16 and B.dtype == torch.float16:
        return wmma_matmul(A, B, out_dtype=torch.float16)
    if A.dtype != torch.float32 or B.dtype != torch.float32:
        raise RuntimeError("matmul expects two float32 (or two float16) tensors")
    return _gemm_f32_nn(_rows_dense(A), _rows_dense(B))


def _rows_dense(t: torch.Tensor) -> torch.Tensor:
    """t itself when its rows can be addressed as row r at r * stride(0) with
    unit column stride and non-overlapping rows (stride(0) >= row length, or a
    single row); otherwise a contiguous copy. Broadcast views (expand(),
    stride(0) == 0) and other overlapping layouts are copied."""
    rows, cols = t.shape
    if t.stride(1) == 1 and (rows <= 1 or t.stride(0) >= cols):
        return t
    return t.contiguous()


# fp32 products of at least this many multiply-adds (and K % 4 == 0) transpose
# B once into W[N, K] and run on the fp32 MFMA GEMM, 2-5x the SIMT kernel's
# rate on B[K, N]; smaller ones take the SIMT kernel in one launch.
_F32_MFMA_MIN_MACS = 1 << 18


def _gemm_f32_nn(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """C[M,N] = A[M,K] . B[K,N] in fp32 (row-major, unit column stride)."""
    M, K = A.shape
    N = B.shape[1]
    C = torch.empty((M, N), dtype=torch.float32, device=A.device)
    if M == 0 or N == 0:
        return C
    s = _stream(A)
    # single-row operands may carry any stride(0); use the dense row length
    lda = A.stride(0) if M > 1 else K
    ldb = B.stride(0) if K > 1 else N
    if K % 4 == 0 and M * N * K >= _F32_MFMA_MIN_MACS:
        bt = torch.empty((N, K), dtype=torch.float32, device=A.device)
        if ldb == N:
            L.call("zk_transpose_0213", _p(B), _p(bt), 1, K, N, 1, L.ZK_F32, s)
        else:  # strided rows: transpose the dense copy
            L.call("zk_transpose_0213", _p(B.contiguous()), _p(bt), 1, K, N, 1, L.ZK_F32, s)
        ws = gemm_workspace(M, N, K, L.ZK_F32, A.device)
        L.call("zk_gemm_f32_ws", _p(A), _p(bt), _p(C), M, N, K, lda, K, N, 1, *_ws_args(ws), s)
    else:
        L.call("zk_gemm_f32", _p(A), _p(B), _p(C), M, N, K, lda, ldb, N, 0, s)
    return C


_ACT_EPI = {
    None: L.ZK_EPI_BIAS,
    "gelu": L.ZK_EPI_BIAS_GELU_ERF,
    "gelu_erf": L.ZK_EPI_BIAS_GELU_ERF,
    "gelu_tanh": L.ZK_EPI_BIAS_GELU_TANH,
    "relu": L.ZK_EPI_BIAS_RELU,
}


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
           activation: str | None = None,
           residual: torch.Tensor | None = None) -> torch.Tensor:
    """y = act(x . weight^T + bias) [+ residual], torch Linear layout
    weight[N, K]. fp16 runs on the MFMA kernel with the epilogue fused
    (Linear+GELU: fused_gemm_epilogue_gelu, core/src/fused_kernels.cu:317-330);
    fp32 runs zk_linear_f32, the fp32 GEMM with the same epilogues fused."""
    _need_cuda(x, weight, bias, residual)
    if weight.dim() != 2 or x.shape[-1] != weight.shape[1]:
        raise RuntimeError("linear: weight must be [out_features, in_features]")
    if activation not in _ACT_EPI:
        raise RuntimeError(f"linear: unsupported activation {activation!r}")
    if residual is not None and activation is not None:
        raise RuntimeError("linear: residual and activation cannot be combined")
    lead = x.shape[:-1]
    K = x.shape[-1]
    N = weight.shape[0]
    x2 = x.reshape(-1, K)
    if x.dtype == torch.float16:
        if weight.dtype != torch.float16:
            raise RuntimeError("linear: fp16 input needs an fp16 weight")
        b = bias
        if b is None and (activation is not None or residual is not None):
            b = torch.zeros(N, dtype=torch.float16, device=x.device)
        if b is not None:
            if b.numel() != N or b.dtype != torch.float16:
                raise RuntimeError("linear: bias must be [out_features] fp16")
            b = b.contiguous()
        epi = L.ZK_EPI_NONE if b is None else _ACT_EPI[activation]
        res2 = None
        if residual is not None:
            res2 = residual.reshape(-1, N)
            if res2.dtype != torch.float16 or res2.shape[0] != x2.shape[0]:
                raise RuntimeError("linear: residual must be [..., out_features] fp16")
            epi = L.ZK_EPI_BIAS_RESIDUAL
        x2 = x2 if x2.stride(1) == 1 else x2.contiguous()
        w = weight if weight.stride(1) == 1 else weight.contiguous()
        if x2.shape[0] == 0:
            return torch.empty(*lead, N, dtype=torch.float16, device=x.device)
        y = _gemm_f16_nt(x2, w, torch.float16, bias=b, residual=res2, epilogue=epi)
        return y.reshape(*lead, N)
    if x.dtype != torch.float32 or weight.dtype != torch.float32:
        raise RuntimeError("linear expects float32 or float16 tensors")
    b = bias
    if b is None and (activation is not None or residual is not None):
        b = torch.zeros(N, dtype=torch.float32, device=x.device)
    if b is not None:
        if b.numel() != N:
            raise RuntimeError("linear: bias must be [out_features]")
        b = b.to(torch.float32).contiguous()
    epi = L.ZK_EPI_NONE if b is None else _ACT_EPI[activation]
    res2 = None
    if residual is not None:
        res2 = residual.reshape(-1, N).to(torch.float32).contiguous()
        if res2.shape[0] != x2.shape[0]:
            raise RuntimeError("linear: residual must be [..., out_features]")
        epi = L.ZK_EPI_BIAS_RESIDUAL
    x2 = x2.contiguous()
    w = weight.contiguous()
    M = x2.shape[0]
    y = torch.empty((M, N), dtype=torch.float32, device=x.device)
    if M:
        ws = gemm_workspace(M, N, K, L.ZK_F32, x.device)
        L.call("zk_linear_f32", _p(x2), _p(w), _p(y), M, N, K, K, K, N, _p(b), _p(res2), N, epi,
               *_ws_args(ws), _stream(x2))
    return y.reshape(*lead, N)


# --------------------------------------------------------------- attention --
def _mask_arg(attn_mask: torch.Tensor, B: int, H: int, Sq: int, Sk: int):
    """(uint8 tensor, (batch, head, query) byte strides) for a boolean mask
    broadcastable to [B, H, Sq, Sk]: keys contiguous, rows 4-byte aligned and
    padded to a multiple of 4 keys (copied only when the given layout is not
    already so); broadcast dimensions get stride 0."""
    if attn_mask.dtype != torch.bool:
        raise RuntimeError("flash_attention: attn_mask must be boolean (True = attend); "
                           "additive float masks are not supported")
    if attn_mask.dim() > 4:
        raise RuntimeError("flash_attention: attn_mask has more than 4 dimensions")
    m = attn_mask.reshape((1,) * (4 - attn_mask.dim()) + tuple(attn_mask.shape))
    for have, want in zip(m.shape, (B, H, Sq, Sk)):
        if have not in (1, want):
            raise RuntimeError(f"flash_attention: attn_mask {tuple(attn_mask.shape)} does not "
                               f"broadcast to {(B, H, Sq, Sk)}")
    if m.shape[3] != Sk:
        m = m.expand(*m.shape[:3], Sk)
    m = m.view(torch.uint8)
    ok = (m.stride(3) == 1 and Sk % 4 == 0 and m.data_ptr() % 4 == 0 and
          all(m.stride(i) % 4 == 0 or m.shape[i] == 1 for i in range(3)))
    if not ok:
        skp = (Sk + 3) // 4 * 4
        dense = torch.zeros((*m.shape[:3], skp), dtype=torch.uint8, device=m.device)
        dense[..., :Sk] = m
        m = dense
    strides = [0 if m.shape[i] == 1 else m.stride(i) for i in range(3)]
    return m, strides


def flash_attention(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor,
                    key_padding_lengths: torch.Tensor | None = None,
                    scale: float | None = None,
                    attn_mask: torch.Tensor | None = None) -> torch.Tensor:
    """softmax(scale . Q K^T) V over [batch, heads, seq, head_dim] tensors,
    non-causal (reference flash_attention_forward, flash_attention.cu:327-340,
    scale 1/sqrt(head_dim)). `key_padding_lengths` (int, [batch]) masks keys
    j >= length; `attn_mask` (bool, broadcastable to [batch, heads, seq_q,
    seq_k], True = attend: scaled_dot_product_attention's boolean mask) masks
    any (query, key) pair; both may be given. Masked keys get probability
    exactly 0 and a query with no key left returns 0. fp32 and fp16; any
    head_dim up to 128 (HEAD_DIM_MAX, flash_attention.cu:26); fp16 head_dims
    that are not a multiple of 8 are zero-padded to one."""
    if not Q.is_cuda:
        raise RuntimeError("Q must be CUDA tensor")
    _need_cuda(Q, K, V, key_padding_lengths, attn_mask)
    if Q.dim() != 4:
        raise RuntimeError("Q must be 4D [batch, heads, seq, dim]")
    if K.dim() != 4 or V.dim() != 4:
        raise RuntimeError("K and V must be 4D [batch, heads, seq, dim]")
    B, H, Sq, D = Q.shape
    Sk = K.shape[2]
    if K.shape != (B, H, Sk, D) or V.shape != (B, H, Sk, D):
        raise RuntimeError("K and V must be [batch, heads, seq_k, dim] matching Q")
    if not (Q.dtype == K.dtype == V.dtype):
        raise RuntimeError("Q, K and V must share a dtype")
    dt = _float_dtype(Q, "flash_attention")

    def lastdim(t):
        return t if t.stride(3) == 1 else t.contiguous()

    if D > 128:
        raise RuntimeError(f"flash_attention: head_dim {D} > 128 is not supported")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    lens = None
    if key_padding_lengths is not None:
        lens = key_padding_lengths.to(device=Q.device, dtype=torch.int32).contiguous()
        if lens.numel() != B:
            raise RuntimeError("key_padding_lengths must have one entry per batch")
    mask = None if attn_mask is None else _mask_arg(attn_mask, B, H, Sq, Sk)
    if dt == L.ZK_F16 and D % 8:
        # zero columns add nothing to Q.K^T; V's give output columns dropped below
        Dp = (D + 7) // 8 * 8
        pad = lambda t: torch.nn.functional.pad(t, (0, Dp - D))  # noqa: E731
        O = torch.empty((B, H, Sq, Dp), dtype=Q.dtype, device=Q.device)
        Qp, Kp, Vp = pad(Q), pad(K), pad(V)
        _attn_call(Qp, Kp, Vp, O, B, H, Sq, Sk, Dp,
                   [*Qp.stride()[:3], *Kp.stride()[:3], *Vp.stride()[:3], *O.stride()[:3]],
                   lens, scale, dt, mask)
        return O[..., :D].contiguous()
    Q, K, V = lastdim(Q), lastdim(K), lastdim(V)
    O = torch.empty((B, H, Sq, D), dtype=Q.dtype, device=Q.device)
    return _attn_call(Q, K, V, O, B, H, Sq, Sk, D,
                      [*Q.stride()[:3], *K.stride()[:3], *V.stride()[:3], *O.stride()[:3]],
                      lens, scale, dt, mask)


def _attn_call(Q, K, V, O, B, H, Sq, Sk, D, strides, lens, scale, dt, mask=None):
    if dt == L.ZK_F16 and (any(s % 8 for s in strides) or
                           any(t.data_ptr() % 16 for t in (Q, K, V, O))):
        Q, K, V = Q.contiguous(), K.contiguous(), V.contiguous()
        strides = [*Q.stride()[:3], *K.stride()[:3], *V.stride()[:3], *O.stride()[:3]]
    if mask is None:
        L.call("zk_flash_attn_fwd", _p(Q), _p(K), _p(V), _p(O), B, H, Sq, Sk, D,
               L.strides_arg(strides), _p(lens), float(scale), dt, _stream(Q))
    else:
        m, ms = mask
        L.call("zk_flash_attn_fwd_masked", _p(Q), _p(K), _p(V), _p(O), B, H, Sq, Sk, D,
               L.strides_arg(strides), _p(lens), _p(m), L.strides_arg(ms), float(scale), dt,
               _stream(Q))
    return O


# ------------------------------------------------------------------- int8 ---
def quantize_int8(x: torch.Tensor, scale: float) -> torch.Tensor:
    """q = clamp(round_half_even(x / scale), -128, 127) as int8
    (quantize_f32_to_int8_kernel, core/src/cuda_kernels.cu:918-937)."""
    _need_cuda(x)
    dt = _float_dtype(x, "quantize_int8")
    x = x.contiguous()
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    L.call("zk_quantize_i8", _p(x), _p(q), x.numel(), float(scale), dt, _stream(x))
    return q


def int8_matmul(a_q: torch.Tensor, w_q: torch.Tensor) -> torch.Tensor:
    """Raw int32 accumulators a_q[M,K] . w_q[N,K]^T (int8 operands)."""
    _need_cuda(a_q, w_q)
    if a_q.dtype != torch.int8 or w_q.dtype != torch.int8:
        raise RuntimeError("int8_matmul expects int8 tensors")
    if a_q.dim() != 2 or w_q.dim() != 2 or a_q.shape[1] != w_q.shape[1]:
        raise RuntimeError("int8_matmul: expected a[M,K] and w[N,K]")
    a_q, w_q = _pad_k(a_q, 16), _pad_k(w_q, 16)
    M, K = a_q.shape
    N = w_q.shape[0]
    out = torch.empty((M, N), dtype=torch.int32, device=a_q.device)
    if M and N:
        L.call("zk_gemm_i8", _p(a_q), _p(w_q), _p(out), M, N, K, a_q.stride(0),
               w_q.stride(0), out.stride(0), 1.0, None, None, None, 0, L.ZK_EPI_NONE,
               L.ZK_I32, _stream(a_q))
    return out


def int8_linear(a_q: torch.Tensor, w_q: torch.Tensor, s_x: float, s_w: torch.Tensor,
                bias: torch.Tensor | None = None, activation: str | None = None,
                residual: torch.Tensor | None = None,
                out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """y = act((a_q . w_q^T) * s_x * s_w[n] + bias) [+ residual] with int32
    accumulation and the dequantisation fused into the epilogue."""
    _need_cuda(a_q, w_q, s_w, bias, residual)
    if a_q.dtype != torch.int8 or w_q.dtype != torch.int8:
        raise RuntimeError("int8_linear expects int8 operands")
    if a_q.dim() != 2 or w_q.dim() != 2 or a_q.shape[1] != w_q.shape[1]:
        raise RuntimeError("int8_linear: expected a[M,K] and w[N,K]")
    if out_dtype not in (torch.float16, torch.float32):
        raise RuntimeError("int8_linear: out_dtype must be float16 or float32")
    if activation not in _ACT_EPI:
        raise RuntimeError(f"int8_linear: unsupported activation {activation!r}")
    a_q, w_q = _pad_k(a_q, 16), _pad_k(w_q, 16)
    M, K = a_q.shape
    N = w_q.shape[0]
    s_w = s_w.to(torch.float32).contiguous()
    if s_w.numel() != N:
        raise RuntimeError("int8_linear: s_w must be [out_features]")
    b = bias
    if b is None and (activation is not None or residual is not None):
        b = torch.zeros(N, dtype=out_dtype, device=a_q.device)
    if b is not None:
        b = b.to(out_dtype).contiguous()
    epi = L.ZK_EPI_NONE if b is None else _ACT_EPI[activation]
    ldr = 0
    if residual is not None:
        residual = residual.to(out_dtype).contiguous()
        ldr = residual.stride(0)
        epi = L.ZK_EPI_BIAS_RESIDUAL
    out = torch.empty((M, N), dtype=out_dtype, device=a_q.device)
    if M and N:
        L.call("zk_gemm_i8", _p(a_q), _p(w_q), _p(out), M, N, K, a_q.stride(0),
               w_q.stride(0), out.stride(0), float(s_x), _p(s_w), _p(b), _p(residual), ldr,
               epi, _DT[out_dtype], _stream(a_q))
    return out


def int8_linear_q8(a_q: torch.Tensor, w_q: torch.Tensor, s_x: float, s_w: torch.Tensor,
                   bias: torch.Tensor | None, activation: str | None,
                   s_out: float) -> torch.Tensor:
    """quantize_int8(int8_linear(a_q, w_q, s_x, s_w, bias, activation), s_out)
    in one kernel: the dequantised, biased, activated fp16 value is
    re-quantised in the GEMM epilogue (int8 out, no fp16 intermediate)."""
    _need_cuda(a_q, w_q, s_w, bias)
    if a_q.dtype != torch.int8 or w_q.dtype != torch.int8:
        raise RuntimeError("int8_linear_q8 expects int8 operands")
    if a_q.dim() != 2 or w_q.dim() != 2 or a_q.shape[1] != w_q.shape[1]:
        raise RuntimeError("int8_linear_q8: expected a[M,K] and w[N,K]")
    if activation not in _ACT_EPI:
        raise RuntimeError(f"int8_linear_q8: unsupported activation {activation!r}")
    a_q, w_q = _pad_k(a_q, 16), _pad_k(w_q, 16)
    M, K = a_q.shape
    N = w_q.shape[0]
    s_w = s_w.to(torch.float32).contiguous()
    if s_w.numel() != N:
        raise RuntimeError("int8_linear_q8: s_w must be [out_features]")
    b = bias
    if b is None and activation is not None:
        b = torch.zeros(N, dtype=torch.float16, device=a_q.device)
    if b is not None:
        b = b.to(torch.float16).contiguous()
    epi = L.ZK_EPI_NONE if b is None else _ACT_EPI[activation]
    out = torch.empty((M, N), dtype=torch.int8, device=a_q.device)
    if M and N:
        L.call("zk_gemm_i8_requant", _p(a_q), _p(w_q), _p(out), M, N, K, a_q.stride(0),
               w_q.stride(0), out.stride(0), float(s_x), _p(s_w), _p(b), epi, float(s_out),
               _stream(a_q))
    return out


__all__ = [
    "relu", "gelu", "layernorm", "matmul", "flash_attention", "wmma_matmul",
    "add_layernorm", "layernorm_add", "add_layernorm_q8", "bias_gelu", "linear", "transpose_f16",
    "quantize_int8", "int8_matmul", "int8_linear", "int8_linear_q8",
]

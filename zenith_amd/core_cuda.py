"""GPU-resident tensor API of the reference's ``_zenith_core.cuda`` module, over
the HIP kernels of libzenith_hip.so.

Mirrors python/src/bindings.cpp:1367-2009 (the transformer/BERT operations on
GpuTensor) and the GpuTensor class with its factories (:694-781): the same
function names, positional arguments, defaults, fp32 GpuTensor inputs and
outputs, and RuntimeError on the same preconditions. It is the API behind the
reference's published BERT comparator (benchmarks/bert_hybrid.py:96-146);
a caller switches with ``from zenith_amd import core_cuda as cuda``.

It also carries what the GPU branches of the reference's ONNX operators call
(zenith/execution/operators/activation_ops.py:52-181, math_ops.py:83-190,
context.py:56-182): is_available, to_gpu, to_numpy, relu_gpu, sigmoid_gpu,
tanh_gpu, softmax_gpu, gelu_gpu and the NumPy-array functions matmul and add,
so those branches reach the HIP kernels when this module stands in for
``_zenith_core.cuda``. (In the reference, to_numpy is only a GpuTensor method
and sigmoid_gpu / tanh_gpu are not bound, so those branches always end in the
operators' NumPy fallbacks.) The NumPy-array functions gelu, layernorm and
softmax (bindings.cpp:2010-2131) are here too; the cuDNN convolution, pooling
and batch-norm functions are not (no CNN path in this build).

Differences from the reference, by design:
  - every operation runs a kernel of libzenith_hip.so on torch's current
    stream (no cuBLAS; the `*_fp16_gpu` functions convert with zk_convert,
    run the fp16 kernel and convert back, as the reference does with its
    conversion kernels);
  - device memory comes from torch's caching allocator, so the fp16 staging
    buffers are not cudaMalloc'd per call (bindings.cpp:1811-1849) and not
    held in process-wide statics (:1740-1760);
  - softmax is the row softmax without the reference kernel's write race
    (core/src/cuda_kernels.cu:220-246: every thread of the block writes the
    row before one normalises it).
Nothing here falls back to torch arithmetic: the library must load.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import _lib as L
from .zenith_cuda import _gemm_f32_nn, _pad_k, _ws_args, gemm_workspace

F32, F16 = torch.float32, torch.float16


class GpuTensor:
    """fp32 tensor resident on the GPU (bindings.cpp:694-755). A default
    constructed GpuTensor is invalid, like the reference's."""

    __slots__ = ("_t",)

    def __init__(self, tensor: torch.Tensor | None = None):
        if tensor is not None:
            if tensor.dtype != F32 or tensor.device.type != "cuda":
                raise RuntimeError("GpuTensor holds float32 data on the GPU")
            tensor = tensor.contiguous()
        self._t = tensor

    def is_valid(self) -> bool:
        return self._t is not None

    def numel(self) -> int:
        return int(self._t.numel()) if self._t is not None else 0

    def size_bytes(self) -> int:
        return 4 * self.numel()

    def ndim(self) -> int:
        return self._t.dim() if self._t is not None else 0

    def dim(self, axis: int) -> int:
        if self._t is None:
            raise RuntimeError("Invalid GpuTensor")
        if axis < 0 or axis >= self._t.dim():
            raise RuntimeError("Axis out of range")
        return int(self._t.shape[axis])

    @property
    def shape(self) -> tuple:
        return tuple(self._t.shape) if self._t is not None else ()

    def to_numpy(self) -> np.ndarray:
        if self._t is None:
            raise RuntimeError("Invalid GpuTensor")
        return self._t.cpu().numpy()

    @property
    def tensor(self) -> torch.Tensor:
        """The underlying torch tensor (device memory; no copy)."""
        if self._t is None:
            raise RuntimeError("Invalid GpuTensor")
        return self._t

    def __repr__(self) -> str:
        if self._t is None:
            return "GpuTensor(invalid)"
        return "GpuTensor(shape=[" + ", ".join(str(d) for d in self._t.shape) + "], device=cuda)"


# ------------------------------------------------------------- factories ---
def to_gpu(array) -> GpuTensor:
    """Copy a NumPy array to a float32 GpuTensor (bindings.cpp:760-771)."""
    if not torch.cuda.is_available():
        raise RuntimeError("to_gpu: no GPU is visible")
    a = np.ascontiguousarray(np.asarray(array, dtype=np.float32))
    return GpuTensor(torch.from_numpy(a).to("cuda"))


def empty(shape) -> GpuTensor:
    """Uninitialised float32 GpuTensor (bindings.cpp:773-781)."""
    if not torch.cuda.is_available():
        raise RuntimeError("empty: no GPU is visible")
    return GpuTensor(torch.empty(tuple(int(d) for d in shape), dtype=F32, device="cuda"))


def sync() -> None:
    """Wait for all queued GPU work (bindings.cpp:689-691)."""
    torch.cuda.synchronize()


def is_available() -> bool:
    """True when a GPU is visible and the HIP kernel library loads
    (bindings.cpp:684-686)."""
    if not torch.cuda.is_available():
        return False
    try:
        L.load()
    except RuntimeError:
        return False
    return True


def memory_stats() -> dict:
    """Device-memory pool statistics under the reference's keys
    (bindings.cpp:825-836, pool of core/include/zenith/gpu_tensor.hpp:26-95),
    read from torch's caching allocator, which plays that pool's part here:
    allocations = device allocations made (pool misses), cache_hits =
    requests served from the cache, cache_returns = blocks given back to the
    cache, total_allocated = bytes ever obtained from the device."""
    st = torch.cuda.memory_stats() if torch.cuda.is_available() else {}
    requests = int(st.get("allocation.all.allocated", 0))
    segments = int(st.get("segment.all.allocated", 0))
    return {
        "allocations": segments,
        "cache_hits": max(requests - segments, 0),
        "cache_returns": int(st.get("allocation.all.freed", 0)),
        "total_allocated": int(st.get("reserved_bytes.all.allocated", 0)),
    }


def clear_memory_pool() -> None:
    """Return cached, unused device memory (bindings.cpp:838-839)."""
    if torch.cuda.is_available():
        torch.cuda.empty_cache()


def to_numpy(tensor: GpuTensor) -> np.ndarray:
    """Copy a GpuTensor to a new NumPy array; the module-level form the
    ONNX operators' GPU branches call (activation_ops.py:59,88,117,148,181)."""
    if not isinstance(tensor, GpuTensor):
        raise RuntimeError("to_numpy requires a GpuTensor")
    return tensor.to_numpy()


# --------------------------------------------------------------- helpers ---
def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _valid(name: str, *ts: GpuTensor) -> None:
    for t in ts:
        if not isinstance(t, GpuTensor) or not t.is_valid():
            raise RuntimeError(f"{name} requires valid GpuTensors")


def _new(like: torch.Tensor, shape=None, dtype=F32) -> torch.Tensor:
    return torch.empty(like.shape if shape is None else shape, dtype=dtype, device=like.device)


def _to16(t: torch.Tensor) -> torch.Tensor:
    out = _new(t, dtype=F16)
    L.call("zk_convert", t.data_ptr(), out.data_ptr(), t.numel(), L.ZK_F32, L.ZK_F16, _stream(t))
    return out


def _to32(t: torch.Tensor) -> GpuTensor:
    out = _new(t, dtype=F32)
    L.call("zk_convert", t.data_ptr(), out.data_ptr(), t.numel(), L.ZK_F16, L.ZK_F32, _stream(t))
    return GpuTensor(out)


def _attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dtype: int) -> torch.Tensor:
    B, H, S, D = q.shape
    o = _new(q)
    strides = L.strides_arg([*q.stride()[:3], *k.stride()[:3], *v.stride()[:3], *o.stride()[:3]])
    L.call("zk_flash_attn_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, S,
           k.shape[2], D, strides, None, 1.0 / math.sqrt(D), dtype, _stream(q))
    return o


def _qkv4(name: str, Q: GpuTensor, K: GpuTensor, V: GpuTensor):
    _valid(name, Q, K, V)
    if Q.ndim() != 4 or K.ndim() != 4 or V.ndim() != 4:
        raise RuntimeError(f"{name} requires 4D tensors [batch, heads, seq, dim]")
    q, k, v = Q.tensor, K.tensor, V.tensor
    if k.shape != v.shape or q.shape[:2] != k.shape[:2] or q.shape[3] != k.shape[3]:
        raise RuntimeError(f"{name}: Q, K, V shapes do not match")
    return q, k, v


# ------------------------------------------------------------ operations ---
def gelu_gpu(input: GpuTensor) -> GpuTensor:
    """tanh-approximation GELU (gelu_f32, core/src/cuda_kernels.cu:115-126)."""
    _valid("gelu_gpu", input)
    x = input.tensor
    y = _new(x)
    L.call("zk_gelu", x.data_ptr(), None, y.data_ptr(), 1, x.numel(), L.ZK_GELU_TANH, L.ZK_F32,
           _stream(x))
    return GpuTensor(y)


def layernorm_gpu(input: GpuTensor, gamma: GpuTensor, beta: GpuTensor,
                  eps: float = 1e-5) -> GpuTensor:
    """LayerNorm over the last dim of a 2D [batch, hidden] tensor."""
    _valid("layernorm_gpu", input, gamma, beta)
    if input.ndim() != 2:
        raise RuntimeError("layernorm_gpu requires valid 2D GpuTensor [batch, hidden]")
    return _layernorm(input.tensor, None, gamma.tensor, beta.tensor, eps, L.ZK_F32)


def _layernorm(x, r, g, b, eps, dtype):
    rows, hidden = x.shape
    if g.numel() != hidden or b.numel() != hidden:
        raise RuntimeError("layernorm: gamma and beta must have `hidden` elements")
    y = _new(x, dtype=x.dtype)
    L.call("zk_layernorm", x.data_ptr(), None if r is None else r.data_ptr(), g.data_ptr(),
           b.data_ptr(), y.data_ptr(), rows, hidden, float(eps), dtype, _stream(x))
    return GpuTensor(y) if dtype == L.ZK_F32 else y


def matmul_gpu(A: GpuTensor, B: GpuTensor) -> GpuTensor:
    """C[M,N] = A[M,K] @ B[K,N] in fp32."""
    _valid("matmul_gpu", A, B)
    if A.ndim() != 2 or B.ndim() != 2:
        raise RuntimeError("matmul_gpu requires 2D tensors")
    if A.dim(1) != B.dim(0):
        raise RuntimeError("matmul_gpu dimension mismatch")
    return GpuTensor(_matmul_nn(A.tensor, B.tensor))


def _matmul_nn(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    return _gemm_f32_nn(a, b)


def linear_gpu(X: GpuTensor, W: GpuTensor, bias: GpuTensor) -> GpuTensor:
    """Y[M,N] = X[M,K] @ W[N,K]^T + bias[N] in fp32; the bias is added only
    when it is valid with N elements (bindings.cpp:1454-1498)."""
    _valid("linear_gpu", X, W)
    if X.ndim() != 2 or W.ndim() != 2:
        raise RuntimeError("linear_gpu requires 2D tensors")
    x, w = X.tensor, W.tensor
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise RuntimeError("linear_gpu: W.dim(1) must match X.dim(1)")
    y = _new(x, (M, N))
    has_bias = isinstance(bias, GpuTensor) and bias.is_valid() and bias.dim(0) == N
    ws = gemm_workspace(M, N, K, L.ZK_F32, x.device)
    L.call("zk_linear_f32", x.data_ptr(), w.data_ptr(), y.data_ptr(), M, N, K, K, K, N,
           bias.tensor.data_ptr() if has_bias else None, None, 0,
           L.ZK_EPI_BIAS if has_bias else L.ZK_EPI_NONE, *_ws_args(ws), _stream(x))
    return GpuTensor(y)


def softmax_gpu(input: GpuTensor) -> GpuTensor:
    """Row softmax of a 2D [batch, seq_len] tensor."""
    _valid("softmax_gpu", input)
    if input.ndim() != 2:
        raise RuntimeError("softmax_gpu requires valid 2D GpuTensor [batch, seq_len]")
    x = input.tensor
    y = _new(x)
    L.call("zk_softmax", x.data_ptr(), y.data_ptr(), x.shape[0], x.shape[1], L.ZK_F32, _stream(x))
    return GpuTensor(y)


def flash_attention_gpu(Q: GpuTensor, K: GpuTensor, V: GpuTensor) -> GpuTensor:
    """softmax(Q K^T / sqrt(D)) V on [batch, heads, seq, dim] fp32."""
    q, k, v = _qkv4("flash_attention_gpu", Q, K, V)
    return GpuTensor(_attn(q, k, v, L.ZK_F32))


def cublas_attention_gpu(Q: GpuTensor, K: GpuTensor, V: GpuTensor) -> GpuTensor:
    """The same attention as flash_attention_gpu (the reference's cuBLAS
    variant computes the identical function)."""
    q, k, v = _qkv4("cublas_attention_gpu", Q, K, V)
    return GpuTensor(_attn(q, k, v, L.ZK_F32))


def add_2d_gpu(A: GpuTensor, B: GpuTensor) -> GpuTensor:
    """C = A + B for 2D tensors of one shape."""
    _valid("add_2d_gpu", A, B)
    if A.ndim() != 2 or B.ndim() != 2:
        raise RuntimeError("add_2d_gpu requires 2D tensors")
    if A.shape != B.shape:
        raise RuntimeError("add_2d_gpu: shapes differ")
    a, b = A.tensor, B.tensor
    c = _new(a)
    L.call("zk_add", a.data_ptr(), b.data_ptr(), c.data_ptr(), a.shape[0], a.shape[1], a.shape[0],
           L.ZK_F32, _stream(a))
    return GpuTensor(c)


def fused_add_layernorm_gpu(x: GpuTensor, residual: GpuTensor, gamma: GpuTensor,
                            beta: GpuTensor, eps: float = 1e-5) -> GpuTensor:
    """LayerNorm(x + residual) in one kernel."""
    _valid("fused_add_layernorm_gpu", x, residual, gamma, beta)
    if x.ndim() != 2:
        raise RuntimeError("fused_add_layernorm_gpu requires 2D tensor [batch, hidden]")
    if residual.shape != x.shape:
        raise RuntimeError("fused_add_layernorm_gpu: residual must match x")
    return _layernorm(x.tensor, residual.tensor, gamma.tensor, beta.tensor, eps, L.ZK_F32)


def fused_bias_gelu_gpu(input: GpuTensor, bias: GpuTensor) -> GpuTensor:
    """GELU(input + bias) (tanh form, core/src/fused_kernels.cu:47-62)."""
    _valid("fused_bias_gelu_gpu", input, bias)
    if input.ndim() != 2:
        raise RuntimeError("fused_bias_gelu_gpu requires 2D tensor [batch, features]")
    x, b = input.tensor, bias.tensor
    rows, cols = x.shape
    if b.numel() != cols:
        raise RuntimeError("fused_bias_gelu_gpu: bias must have `features` elements")
    y = _new(x)
    L.call("zk_gelu", x.data_ptr(), b.data_ptr(), y.data_ptr(), rows, cols, L.ZK_GELU_TANH,
           L.ZK_F32, _stream(x))
    return GpuTensor(y)


def _transpose(name, input: GpuTensor, d0, d1, d2, d3) -> GpuTensor:
    _valid(name, input)
    if input.numel() != d0 * d1 * d2 * d3:
        raise RuntimeError(f"{name}: shape does not match the tensor's size")
    x = input.tensor
    y = _new(x, (d0, d2, d1, d3))
    L.call("zk_transpose_0213", x.data_ptr(), y.data_ptr(), d0, d1, d2, d3, L.ZK_F32, _stream(x))
    return GpuTensor(y)


def transpose_for_attention(input: GpuTensor, batch: int, seq: int, heads: int,
                            dim: int) -> GpuTensor:
    """[B,S,H,D] -> [B,H,S,D]."""
    return _transpose("transpose_for_attention", input, batch, seq, heads, dim)


def transpose_from_attention(input: GpuTensor, batch: int, heads: int, seq: int,
                             dim: int) -> GpuTensor:
    """[B,H,S,D] -> [B,S,H,D]."""
    return _transpose("transpose_from_attention", input, batch, heads, seq, dim)


def reshape_4d_to_2d(input: GpuTensor, batch: int, seq: int, hidden: int) -> GpuTensor:
    """[B,S,H,D] -> [B*S, H*D] as a new tensor (a device-to-device copy)."""
    _valid("reshape_4d_to_2d", input)
    if input.numel() != batch * seq * hidden:
        raise RuntimeError("reshape_4d_to_2d: shape does not match the tensor's size")
    return GpuTensor(input.tensor.reshape(batch * seq, hidden).clone())


# fp16 variants: fp32 in and out, fp16 arithmetic in between
def attention_fp16_gpu(Q: GpuTensor, K: GpuTensor, V: GpuTensor) -> GpuTensor:
    """Attention in fp16 on the matrix cores (bindings.cpp:1731-1788)."""
    q, k, v = _qkv4("attention_fp16_gpu", Q, K, V)
    return _to32(_attn(_to16(q), _to16(k), _to16(v), L.ZK_F16))


def attention_full_fp16_gpu(Q: GpuTensor, K: GpuTensor, V: GpuTensor) -> GpuTensor:
    """Same as attention_fp16_gpu (bindings.cpp:1964-2009)."""
    q, k, v = _qkv4("attention_full_fp16_gpu", Q, K, V)
    return _to32(_attn(_to16(q), _to16(k), _to16(v), L.ZK_F16))


def linear_fp16_gpu(X: GpuTensor, W: GpuTensor, bias: GpuTensor) -> GpuTensor:
    """Y = X @ W^T + bias on the fp16 MFMA GEMM; the fp16 output is converted
    back to fp32 (bindings.cpp:1797-1855)."""
    _valid("linear_fp16_gpu", X, W)
    if X.ndim() != 2 or W.ndim() != 2:
        raise RuntimeError("linear_fp16_gpu requires 2D tensors")
    x, w = X.tensor, W.tensor
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise RuntimeError("linear_fp16_gpu: W.dim(1) must match X.dim(1)")
    has_bias = isinstance(bias, GpuTensor) and bias.is_valid() and bias.dim(0) == N
    x16, w16 = _to16(x), _to16(w)
    b16 = _to16(bias.tensor) if has_bias else None
    y16 = _new(x, (M, N), F16)
    x16, w16 = _pad_k(x16, 8), _pad_k(w16, 8)  # zero columns: K a multiple of 8
    K = x16.shape[1]
    ws = gemm_workspace(M, N, K, L.ZK_F16, x.device)
    L.call("zk_gemm_f16_ws", x16.data_ptr(), w16.data_ptr(), y16.data_ptr(), M, N, K, K, K, N, 1,
           L.ZK_F16, None if b16 is None else b16.data_ptr(), None, 0,
           L.ZK_EPI_BIAS if has_bias else L.ZK_EPI_NONE, *_ws_args(ws), _stream(x))
    return _to32(y16)


def gelu_fp16_gpu(input: GpuTensor) -> GpuTensor:
    """tanh GELU in fp16 (fp32 math, fp16 rounding; fp16_kernels.cu:128-147)."""
    _valid("gelu_fp16_gpu", input)
    x16 = _to16(input.tensor)
    y16 = torch.empty_like(x16)
    L.call("zk_gelu", x16.data_ptr(), None, y16.data_ptr(), 1, x16.numel(), L.ZK_GELU_TANH,
           L.ZK_F16, _stream(x16))
    return _to32(y16)


def layernorm_fp16_gpu(input: GpuTensor, gamma: GpuTensor, beta: GpuTensor,
                       eps: float = 1e-5) -> GpuTensor:
    """fp16 LayerNorm with fp32 statistics (fp16_kernels.cu:154-265)."""
    _valid("layernorm_fp16_gpu", input, gamma, beta)
    if input.ndim() != 2:
        raise RuntimeError("layernorm_fp16_gpu requires 2D input")
    y16 = _layernorm(_to16(input.tensor), None, _to16(gamma.tensor), _to16(beta.tensor), eps,
                     L.ZK_F16)
    return _to32(y16)


def add_fp16_gpu(a: GpuTensor, b: GpuTensor) -> GpuTensor:
    """Elementwise a + b in fp16 (fp16_kernels.cu:267-280)."""
    _valid("add_fp16_gpu", a, b)
    if a.numel() != b.numel():
        raise RuntimeError("add_fp16_gpu: sizes differ")
    a16, b16 = _to16(a.tensor), _to16(b.tensor)
    c16 = torch.empty_like(a16)
    L.call("zk_add", a16.data_ptr(), b16.data_ptr(), c16.data_ptr(), 1, a16.numel(), 1, L.ZK_F16,
           _stream(a16))
    return _to32(c16)


# ------------------------------------------------- activations (any rank) --
def _unary(name: str, entry: str, input: GpuTensor) -> GpuTensor:
    _valid(name, input)
    x = input.tensor
    y = _new(x)
    L.call(entry, x.data_ptr(), y.data_ptr(), x.numel(), L.ZK_F32, _stream(x))
    return GpuTensor(y)


def relu_gpu(input: GpuTensor) -> GpuTensor:
    """max(x, 0) (bindings.cpp:1224-1246). Any rank: the reference's 4D
    requirement comes from its cuDNN tensor descriptor, not from ReLU."""
    return _unary("relu_gpu", "zk_relu", input)


def sigmoid_gpu(input: GpuTensor) -> GpuTensor:
    """1 / (1 + exp(-x)): the function the ONNX Sigmoid operator's GPU branch
    calls (activation_ops.py:82-91); not bound in the reference."""
    return _unary("sigmoid_gpu", "zk_sigmoid", input)


def tanh_gpu(input: GpuTensor) -> GpuTensor:
    """tanh(x): the function the ONNX Tanh operator's GPU branch calls
    (activation_ops.py:111-120); not bound in the reference."""
    return _unary("tanh_gpu", "zk_tanh", input)


def add_gpu(a: GpuTensor, b: GpuTensor) -> GpuTensor:
    """a + b for tensors of one shape (bindings.cpp:1313-1337; any rank, the
    4D requirement there is cuDNN's)."""
    _valid("add_gpu", a, b)
    if a.shape != b.shape:
        raise RuntimeError("add_gpu: shapes differ")
    x, z = a.tensor, b.tensor
    c = _new(x)
    L.call("zk_add", x.data_ptr(), z.data_ptr(), c.data_ptr(), 1, x.numel(), 1, L.ZK_F32,
           _stream(x))
    return GpuTensor(c)


# -------------------------------------------- NumPy-array interface ---
# NumPy float32 in, NumPy float32 out; each call uploads its inputs, runs the
# kernel and copies the result back (bindings.cpp:631-682, 842-870,
# 1117-1150, 2010-2131).
def _host(name: str, array, ndim: int | None) -> torch.Tensor:
    if not torch.cuda.is_available():
        raise RuntimeError(f"{name}: no GPU is visible")
    a = np.ascontiguousarray(np.asarray(array, dtype=np.float32))
    if ndim is not None and a.ndim != ndim:
        raise RuntimeError(f"{name} requires a {ndim}D array")
    return torch.from_numpy(a).to("cuda")


def matmul(A, B) -> np.ndarray:
    """C = A @ B for 2D float32 arrays (bindings.cpp:631-682)."""
    a, b = _host("matmul", A, 2), _host("matmul", B, 2)
    if a.shape[1] != b.shape[0]:
        raise RuntimeError("Inner dimensions do not match")
    return _matmul_nn(a, b).cpu().numpy()


def add(a, b) -> np.ndarray:
    """a + b for float32 arrays of one shape (bindings.cpp:1117-1150)."""
    x, z = _host("add", a, None), _host("add", b, None)
    if x.shape != z.shape:
        raise RuntimeError("add requires arrays of one shape")
    return add_gpu(GpuTensor(x), GpuTensor(z)).to_numpy()


def relu(input) -> np.ndarray:
    """max(x, 0) of a float32 array (bindings.cpp:842-870)."""
    return relu_gpu(GpuTensor(_host("relu", input, None))).to_numpy()


def gelu(input) -> np.ndarray:
    """tanh GELU of a 2D float32 array (bindings.cpp:2017-2046)."""
    return gelu_gpu(GpuTensor(_host("gelu", input, 2))).to_numpy()


def layernorm(input, gamma, beta, eps: float = 1e-5) -> np.ndarray:
    """LayerNorm over the last dim of a 2D float32 array (bindings.cpp:2050-2094)."""
    x = _host("layernorm", input, 2)
    g, b = _host("layernorm", gamma, None), _host("layernorm", beta, None)
    return _layernorm(x, None, g, b, eps, L.ZK_F32).to_numpy()


def softmax(input) -> np.ndarray:
    """Row softmax of a 2D float32 array (bindings.cpp:2097-2131)."""
    return softmax_gpu(GpuTensor(_host("softmax", input, 2))).to_numpy()


__all__ = [
    "GpuTensor", "to_gpu", "to_numpy", "empty", "sync", "is_available", "memory_stats",
    "clear_memory_pool",
    "gelu_gpu", "layernorm_gpu", "matmul_gpu", "linear_gpu", "softmax_gpu",
    "flash_attention_gpu", "cublas_attention_gpu", "add_2d_gpu",
    "fused_add_layernorm_gpu", "fused_bias_gelu_gpu",
    "transpose_for_attention", "transpose_from_attention", "reshape_4d_to_2d",
    "attention_fp16_gpu", "attention_full_fp16_gpu", "linear_fp16_gpu",
    "gelu_fp16_gpu", "layernorm_fp16_gpu", "add_fp16_gpu",
    "relu_gpu", "sigmoid_gpu", "tanh_gpu", "add_gpu",
    "matmul", "add", "relu", "gelu", "layernorm", "softmax",
]

"""CPU oracle: numpy restatement of the reference's CPU path for the BERT
encoder kernel set. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Every function names the reference code it follows (paths relative to the
vibeswithkk/ZENITH tree). Arithmetic is float32 unless a function says
otherwise; `*_f64` variants exist where a tighter yardstick is useful.
"""

from __future__ import annotations

import math

import numpy as np
from scipy import special

F32 = np.float32

# ----------------------------------------------------------------- GEMM ----


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """C = A @ B in float32 (execute_matmul -> np.matmul,
    zenith/execution/operators/math_ops.py:62-99)."""
    return np.matmul(a.astype(F32, copy=False), b.astype(F32, copy=False))


def matmul_f64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Same product accumulated in float64 (yardstick for fp16-input GEMMs:
    with fp16-representable inputs every product is exact in float64)."""
    return np.matmul(a.astype(np.float64), b.astype(np.float64))


def linear(x: np.ndarray, w: np.ndarray, b: np.ndarray | None = None) -> np.ndarray:
    """y = x . w^T + b with torch-Linear weight layout w[N, K]
    (registry CPU tier: np.dot(x, w.T) + b, zenith/runtime/kernel_registry.py:770-781)."""
    y = np.dot(x.astype(F32, copy=False), w.astype(F32, copy=False).T)
    if b is not None:
        y = y + b.astype(F32, copy=False)
    return y.astype(F32, copy=False)


# ---------------------------------------------------------- activations ----


def relu(x: np.ndarray) -> np.ndarray:
    """max(x, 0) (relu_f32, core/src/cuda_kernels.cu:504-507)."""
    return np.maximum(x, 0).astype(x.dtype, copy=False)


def sigmoid(x: np.ndarray) -> np.ndarray:
    """1 / (1 + exp(-x)) in float32 (execute_sigmoid,
    zenith/execution/operators/activation_ops.py:76-93)."""
    x = x.astype(F32, copy=False)
    with np.errstate(over="ignore"):
        return (F32(1.0) / (F32(1.0) + np.exp(-x))).astype(F32, copy=False)


def tanh(x: np.ndarray) -> np.ndarray:
    """tanh(x) in float32 (execute_tanh, activation_ops.py:105-122)."""
    return np.tanh(x.astype(F32, copy=False))


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) evaluated in float32
    (gelu_kernel core/src/cuda_kernels.cu:115-126; fused_bias_gelu_cpu
    python/src/features_bindings.hpp:59-86). The numpy ONNX op
    (zenith/execution/operators/activation_ops.py:184-186) computes the same
    formula but is promoted to float64 under numpy 2; see gelu_tanh_f64."""
    x = x.astype(F32, copy=False)
    c = F32(0.7978845608028654)
    inner = c * (x + F32(0.044715) * x * x * x)
    return (F32(0.5) * x * (F32(1.0) + np.tanh(inner))).astype(F32, copy=False)


def gelu_tanh_f64(x: np.ndarray) -> np.ndarray:
    """activation_ops.py:184-186 exactly as numpy 2 evaluates it (float64)."""
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x**3)))


def gelu_erf(x: np.ndarray) -> np.ndarray:
    """Exact GELU 0.5 x (1 + erf(x / sqrt(2))) with scipy's erf
    (Erf op zenith/execution/operators/math_ops.py:361-378; exact-GELU primitive
    zenith/jax/primitives.py:566-586)."""
    x = x.astype(F32, copy=False)
    return (F32(0.5) * x * (F32(1.0) + special.erf(x * F32(1.0 / math.sqrt(2.0))).astype(F32))
            ).astype(F32, copy=False)


def bias_gelu(x: np.ndarray, bias: np.ndarray | None, approximate: str = "tanh") -> np.ndarray:
    """GELU(x + bias[col]) (fused_bias_gelu_cpu, features_bindings.hpp:59-86;
    erf variant for BERT's hidden_act='gelu')."""
    v = x.astype(F32, copy=False)
    if bias is not None:
        v = v + bias.astype(F32, copy=False)
    return gelu_tanh(v) if approximate == "tanh" else gelu_erf(v)


def softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """max-subtracted softmax (softmax_f32 core/src/cpu_kernels.cpp:382-408;
    execute_softmax zenith/execution/operators/activation_ops.py:126-157)."""
    x = x.astype(F32, copy=False)
    e = np.exp(x - np.max(x, axis=axis, keepdims=True))
    return (e / np.sum(e, axis=axis, keepdims=True)).astype(F32, copy=False)


# --------------------------------------------------------------- norms -----


def layernorm(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """(x - mean) / sqrt(var + eps) * gamma + beta over the last axis,
    population variance, two-pass (execute_layer_normalization,
    zenith/execution/operators/norm_ops.py:73-90)."""
    x = x.astype(F32, copy=False)
    mean = np.mean(x, axis=-1, keepdims=True)
    var = np.var(x, axis=-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + F32(eps))
    return (y * gamma.astype(F32, copy=False) + beta.astype(F32, copy=False)).astype(F32, copy=False)


def add_layernorm(x: np.ndarray, residual: np.ndarray, gamma: np.ndarray, beta: np.ndarray,
                  eps: float = 1e-5) -> np.ndarray:
    """LayerNorm(x + residual) (fused_add_layernorm_cpu,
    python/src/features_bindings.hpp:116-171: fp32 sum, two-pass variance,
    1/sqrt)."""
    return layernorm(x.astype(F32) + residual.astype(F32), gamma, beta, eps)


def layernorm_add(x: np.ndarray, residual: np.ndarray, gamma: np.ndarray, beta: np.ndarray,
                  eps: float = 1e-5) -> np.ndarray:
    """LayerNorm(x) * gamma + beta + residual, the residual added after the
    normalisation (fused_layernorm_add_kernel, core/src/fused_kernels.cu:
    224-296: statistics of x only, `normalized * gamma[i] + beta[i] +
    res_row[i]` at :292). The reference's GPU kernel takes the single-pass
    variance E[x^2] - mean^2 (:263); this restatement takes the two-pass
    variance of `layernorm` (the two agree to fp32 rounding for
    zero-mean-ish rows, and the two-pass form is the exact one)."""
    return (layernorm(x, gamma, beta, eps) + residual.astype(F32)).astype(F32, copy=False)


# ----------------------------------------------------------- attention -----


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray,
              valid_lens: np.ndarray | None = None, scale: float | None = None,
              dtype=np.float64, mask: np.ndarray | None = None) -> np.ndarray:
    """Dense softmax(scale . Q K^T) V over [B, H, S, D] (reference semantics:
    flash_attention_forward core/src/flash_attention.cu:194-340, scale
    1/sqrt(D) at :330). Key-padding rule of the masked attention primitive
    (zenith/jax/primitives.py:302-310): keys j >= valid_lens[b] get -inf
    logits and probability exactly 0; an all-masked row yields 0. `mask`
    (bool, broadcastable to [B, H, Sq, Sk], True = attend) applies the same
    rule per (query, key) on top of valid_lens.
    Computed in float64 by default."""
    q = q.astype(dtype)
    k = k.astype(dtype)
    v = v.astype(dtype)
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * scale  # [B,H,Sq,Sk]
    if valid_lens is not None:
        lens = np.clip(np.asarray(valid_lens).astype(np.int64), 0, Sk)
        keep = np.arange(Sk)[None, :] < lens[:, None]  # [B, Sk]
        s = np.where(keep[:, None, None, :], s, -np.inf)
    if mask is not None:
        s = np.where(np.asarray(mask, dtype=bool), s, -np.inf)
    with np.errstate(invalid="ignore"):
        m = np.max(s, axis=-1, keepdims=True)
        e = np.exp(s - m)
        p = e / np.sum(e, axis=-1, keepdims=True)
    p = np.nan_to_num(p, nan=0.0)
    return np.matmul(p, v)


# ----------------------------------------------------------------- int8 ----


def quantize_int8(x: np.ndarray, scale) -> np.ndarray:
    """q = clip(round_half_even(x / scale), -128, 127) in float32 arithmetic
    (quantize_to_int8 benchmarks/int8_bench.py:19-27: np.round is
    half-to-even; quantize_f32_to_int8_kernel core/src/cuda_kernels.cu:
    918-937: __float2int_rn then clamp). NaN gives 0: the reference kernel's
    round-to-int conversion returns 0 for NaN before its clamp, and the
    numpy rule's cast of the NaN that np.clip passes through gives 0 on x86
    (a platform-defined cast, so it is written out here)."""
    x = x.astype(F32, copy=False)
    r = np.rint(x / F32(scale))
    r = np.where(np.isnan(r), F32(0), r)
    return np.clip(r, -128, 127).astype(np.int8)


def dequantize_int8(q: np.ndarray, scale) -> np.ndarray:
    """(q - 0) * scale (dequantize_from_int8, int8_bench.py:30-32)."""
    return q.astype(F32) * F32(scale)


def absmax_scale(absmax: float) -> np.float32:
    """Symmetric scale absmax / 127, 1.0 for an all-zero tensor
    (MinMaxCalibrator.compute_params, zenith/optimization/quantization.py:
    101-107; quantize_to_int8 int8_bench.py:22-23)."""
    absmax = F32(absmax)
    return F32(absmax / F32(127.0)) if absmax > 0 else F32(1.0)


class MinMaxObserver:
    """Running min/max over calibration batches (TensorStats.update,
    zenith/optimization/quantization.py:69-72) feeding the symmetric MinMax
    rule (:101-107)."""

    def __init__(self):
        self.min_val = float("inf")
        self.max_val = float("-inf")

    def update(self, t: np.ndarray) -> None:
        self.min_val = min(self.min_val, float(np.min(t)))
        self.max_val = max(self.max_val, float(np.max(t)))

    def scale(self) -> np.float32:
        return absmax_scale(max(abs(self.min_val), abs(self.max_val)))


def quantize_weight_per_channel(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric per-output-channel int8 weights: s_w[n] = max_k |W[n,k]| / 127,
    q = clip(rint(W / s_w[n]), -128, 127) (per-channel FakeQuantize,
    zenith/optimization/qat.py:185-270, with the /127 rule of
    quantization.py:106 and the round-half-even of int8_bench.py:24)."""
    w = w.astype(F32, copy=False)
    amax = np.max(np.abs(w), axis=1)
    s = np.where(amax > 0, amax / F32(127.0), F32(1.0)).astype(F32)
    q = np.clip(np.rint(w / s[:, None]), -128, 127).astype(np.int8)
    return q, s


def int8_matmul_acc(a_q: np.ndarray, w_q: np.ndarray) -> np.ndarray:
    """Exact int32 accumulators a_q[M,K] . w_q[N,K]^T (int8_matmul_reference,
    benchmarks/int8_bench.py:42-45, with the weight in [N,K] layout).
    Computed with float64 BLAS, which is exact here: every product is at most
    2^14 in magnitude and K <= 2^17, so every partial sum is an integer below
    2^31 < 2^53. Small shapes can be cross-checked with `int8_matmul_acc_i64`."""
    K = a_q.shape[1]
    assert K <= 2**17
    acc = np.matmul(a_q.astype(np.float64), w_q.astype(np.float64).T)
    assert np.abs(acc).max(initial=0) < 2**31
    return acc.astype(np.int32)


def int8_matmul_acc_i64(a_q: np.ndarray, w_q: np.ndarray) -> np.ndarray:
    """Same accumulators with plain int64 arithmetic (slow; small shapes)."""
    acc = np.matmul(a_q.astype(np.int64), w_q.astype(np.int64).T)
    assert np.abs(acc).max(initial=0) < 2**31
    return acc.astype(np.int32)


def int8_linear(a_q, w_q, s_x, s_w, bias=None, activation=None, residual=None) -> np.ndarray:
    """y = act(acc * (s_x * s_w[n]) + bias) [+ residual], float32 epilogue
    (int8_matmul_reference int8_bench.py:42-45 followed by the fused
    bias/GELU epilogue of fused_kernels.cu:47-62)."""
    acc = int8_matmul_acc(a_q, w_q).astype(F32)
    y = acc * (F32(s_x) * s_w.astype(F32))[None, :]
    if bias is not None:
        y = y + bias.astype(F32)
    if activation in ("gelu", "gelu_erf"):
        y = gelu_erf(y)
    elif activation == "gelu_tanh":
        y = gelu_tanh(y)
    elif activation == "relu":
        y = relu(y)
    if residual is not None:
        y = y + residual.astype(F32)
    return y.astype(F32, copy=False)

"""The HIP kernels as registry entries, with one calling convention per op
type (what KernelDispatcher passes):

  Linear / Gemm / LinearGelu   fn(x, W[N,K], b=None)
  MatMul                       fn(A[M,K], B[K,N])
  LayerNorm                    fn(x, gamma, beta, eps)
  FusedAddLayerNorm            fn(x, residual, gamma, beta, eps)
  Gelu / FusedBiasGeLU         fn(x) / fn(x, bias)          (approximate= kw)
  Relu                         fn(x)
  Attention / FlashAttention   fn(q, k, v, key_padding_lengths=None, scale=None)
  QKVProjection                fn(x, Wq, bq, Wk, bk, Wv, bv) -> (q, k, v)
  FusedAttentionEpilogue       fn(ctx, residual, Wo, bo, gamma, beta, eps)
  FusedFFN                     fn(x, Wi, bi, Wo2, bo2, gamma, beta, eps)
  QLinear (INT8)               fn(x_q, W_q, s_x, s_w, b=None)

Every entry point runs on the GPU through libzenith_hip.so; tensors on
another device raise RuntimeError (no fallback).
"""

from __future__ import annotations

import torch

from .. import zenith_cuda as zc
from .kernel_registry import KernelRegistry, KernelSpec, Precision

HIP_PRIORITY = 25  # the reference's JIT zenith_cuda tier (kernel_registry.py:215-286)


def _rows(t: torch.Tensor) -> torch.Tensor:
    return t.reshape(-1, t.shape[-1])


def linear(x, w, b=None):
    return zc.linear(x, w, b)


def linear_gelu(x, w, b=None, approximate: str = "none"):
    return zc.linear(x, w, b, activation="gelu_tanh" if approximate == "tanh" else "gelu")


def matmul(a, b):
    return zc.matmul(a, b)


def layernorm(x, gamma, beta, eps: float = 1e-5):
    return zc.layernorm(_rows(x), gamma, beta, eps).view(x.shape)


def add_layernorm(x, residual, gamma, beta, eps: float = 1e-5):
    return zc.add_layernorm(_rows(x), _rows(residual), gamma, beta, eps).view(x.shape)


def gelu(x, approximate: str = "tanh"):
    return zc.gelu(x, approximate=approximate)


def bias_gelu(x, bias, approximate: str = "tanh"):
    return zc.bias_gelu(x, bias, approximate=approximate)


def relu(x):
    return zc.relu(x)


def attention(q, k, v, key_padding_lengths=None, scale=None):
    return zc.flash_attention(q, k, v, key_padding_lengths=key_padding_lengths, scale=scale)


def qkv_projection(x, wq, bq, wk, bk, wv, bv):
    """One GEMM over the concatenated [3H, K] weight, split into q, k, v."""
    w = torch.cat([wq, wk, wv], 0)
    b = None if bq is None else torch.cat([bq, bk, bv], 0)
    y = zc.linear(x, w, b)
    n = wq.shape[0]
    return y[..., :n], y[..., n:2 * n], y[..., 2 * n:]


def attention_epilogue(ctx, residual, wo, bo, gamma, beta, eps: float = 1e-12):
    """LayerNorm(ctx . Wo^T + bo + residual): out-projection GEMM with the
    bias fused, then the fused Add+LayerNorm kernel."""
    return add_layernorm(zc.linear(ctx, wo, bo), residual, gamma, beta, eps)


def ffn(x, wi, bi, wo2, bo2, gamma, beta, eps: float = 1e-12):
    """LayerNorm(GELU(x Wi^T + bi) Wo2^T + bo2 + x): up GEMM with the
    bias + erf-GELU epilogue, down GEMM with bias, fused Add+LayerNorm."""
    u = zc.linear(x, wi, bi, activation="gelu")
    return add_layernorm(zc.linear(u, wo2, bo2), x, gamma, beta, eps)


def qlinear(x_q, w_q, s_x, s_w, b=None):
    """INT8 Linear: int32 accumulation, dequantisation (+ bias) fused."""
    return zc.int8_linear(x_q, w_q, float(s_x), s_w, bias=b)


_TABLE = [
    # name, op types, precisions, fn
    ("hip_linear", ["Linear", "Gemm"], (Precision.FP32, Precision.FP16), linear),
    ("hip_matmul", ["MatMul", "matmul"], (Precision.FP32, Precision.FP16), matmul),
    ("hip_linear_gelu", ["LinearGelu", "FusedLinearGelu"], (Precision.FP32, Precision.FP16),
     linear_gelu),
    ("hip_layernorm", ["LayerNorm", "LayerNormalization", "layer_norm"],
     (Precision.FP32, Precision.FP16), layernorm),
    ("hip_add_layernorm", ["FusedAddLayerNorm", "AddLayerNorm", "Add+LayerNorm"],
     (Precision.FP32, Precision.FP16), add_layernorm),
    ("hip_gelu", ["Gelu", "GELU", "gelu"], (Precision.FP32, Precision.FP16), gelu),
    ("hip_bias_gelu", ["FusedBiasGeLU", "BiasGeLU", "Bias+GELU"],
     (Precision.FP32, Precision.FP16), bias_gelu),
    ("hip_relu", ["Relu", "ReLU", "relu"], (Precision.FP32, Precision.FP16), relu),
    ("hip_flash_attention", ["Attention", "MultiHeadAttention", "FlashAttention",
                             "flash_attention"], (Precision.FP32, Precision.FP16), attention),
    ("hip_qkv_projection", ["QKVProjection"], (Precision.FP32, Precision.FP16), qkv_projection),
    ("hip_attention_epilogue", ["FusedAttentionEpilogue"], (Precision.FP32, Precision.FP16),
     attention_epilogue),
    ("hip_ffn", ["FusedFFN"], (Precision.FP32, Precision.FP16), ffn),
    ("hip_qlinear_int8", ["Linear", "Gemm", "QLinear"], (Precision.INT8,), qlinear),
]


def register_hip_kernels(reg: KernelRegistry) -> None:
    """Register every HIP kernel at priority 25. Raises RuntimeError if the
    library cannot be loaded (there is no other tier)."""
    from .. import _lib

    _lib.load()
    for name, ops, precs, fn in _TABLE:
        for prec in precs:
            reg.register(KernelSpec(name=f"{name}_{prec.value}", op_types=list(ops),
                                    precision=prec, kernel_fn=fn, priority=HIP_PRIORITY,
                                    requires_gpu=True))

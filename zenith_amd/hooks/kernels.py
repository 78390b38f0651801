"""The HIP kernels as registry entries, with one calling convention per op
type (what KernelDispatcher passes):

  Linear / Gemm / LinearGelu   fn(x, W[N,K], b=None)
  MatMul                       fn(A[M,K], B[K,N])
  LayerNorm                    fn(x, gamma, beta, eps)
  FusedAddLayerNorm            fn(x, residual, gamma, beta, eps)
  LayerNormAdd                 fn(x, residual, gamma, beta, eps)   LN(x) + residual
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

import sys

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


def layernorm_add(x, residual, gamma, beta, eps: float = 1e-5):
    """LayerNorm(x) * gamma + beta + residual (the LayerNormAdd node)."""
    return zc.layernorm_add(_rows(x), _rows(residual), gamma, beta, eps).view(x.shape)


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
    ("hip_layernorm_add", ["LayerNormAdd", "FusedLayerNormAdd"],
     (Precision.FP32, Precision.FP16), layernorm_add),
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


def _registry_types(reg, spec_cls, precision_enum):
    """KernelSpec class and Precision enum to build the specs from: the
    explicit arguments, else the ones defined beside the registry's class
    (the reference keeps all three in zenith/runtime/kernel_registry.py), else
    this package's own."""
    mod = sys.modules.get(type(reg).__module__)
    if spec_cls is None:
        spec_cls = getattr(mod, "KernelSpec", None) or KernelSpec
    if precision_enum is None:
        precision_enum = getattr(mod, "Precision", None) or Precision
    return spec_cls, precision_enum


def register_hip_kernels(reg, spec_cls=None, precision_enum=None) -> int:
    """Register every HIP kernel at priority 25 in `reg` and return the
    number of specs registered. Raises RuntimeError if the library cannot be
    loaded (there is no other tier).

    `reg` may be this package's KernelRegistry or the reference's
    (zenith/runtime/kernel_registry.py:92-153). Its get_kernel filters with
    `spec.precision == precision` on its OWN Precision enum, and members of
    two Enum classes never compare equal, so the specs are built from the
    registry's own KernelSpec / Precision (found beside the registry's class,
    or passed explicitly), with each precision matched by its `.value`
    ("fp32", "fp16", "int8"). A precision the caller's enum lacks is
    skipped."""
    from .. import _lib

    _lib.load()
    spec_cls, prec_enum = _registry_types(reg, spec_cls, precision_enum)
    by_value = {m.value: m for m in prec_enum}
    n = 0
    for name, ops, precs, fn in _TABLE:
        for prec in precs:
            target = by_value.get(prec.value)
            if target is None:
                continue
            reg.register(spec_cls(name=f"{name}_{prec.value}", op_types=list(ops),
                                  precision=target, kernel_fn=fn, priority=HIP_PRIORITY,
                                  requires_gpu=True))
            n += 1
    return n

"""torch.fx pattern / replacement pairs that route matched subgraphs to the
HIP kernels.

Mirrors the reference's pattern module (zenith/optimization/fx_patterns.py:
59-229): the same `FXPattern` record, the same pattern functions
(`sdpa_pattern`, `gelu_tanh_pattern`, `layernorm_pattern`) and the same
registry helpers (`get_attention_patterns`, `get_activation_patterns`,
`get_normalization_patterns`, `get_all_patterns`,
`is_zenith_cuda_available`). What changes is where replacements go:

  - `zenith_sdpa_replacement` always calls `zenith_cuda.flash_attention`
    (fp32 or fp16). The reference wrapped it in try/except and fell back to
    F.scaled_dot_product_attention (fx_patterns.py:106-114), which under fp16
    was always taken because its kernel was fp32-only; here an error raises.
  - `zenith_gelu_replacement` and `zenith_layernorm_replacement` call the HIP
    GELU / LayerNorm kernels (the reference rerouted them to F.gelu /
    F.layer_norm, fx_patterns.py:147-179).
  - extra patterns for the fused BERT epilogues: erf-GELU of a Linear
    (Linear+GELU epilogue), LayerNorm of a residual sum (Add+LayerNorm), and
    the functional scaled_dot_product_attention call.

Each replacement calls one `hip_*` leaf registered with torch.fx.wrap, so a
rewritten graph contains one call_function node per fused kernel.
Replacements accept only CUDA tensors (the HIP kernels raise RuntimeError
otherwise); the optimizer rewrites a graph only when its example inputs live
on a GPU.

The causal pattern of the reference (fx_patterns.py:117-131) is not
registered: no causal kernel is part of this library, so a causal subgraph is
left as it is.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable

import torch
import torch.fx
import torch.nn.functional as F

from .. import zenith_cuda


@dataclass
class FXPattern:
    """One subgraph pattern and the callable that replaces it
    (zenith/optimization/fx_patterns.py:59-67)."""

    name: str
    pattern_fn: Callable
    replacement_fn: Callable
    priority: int = 10
    enabled: bool = True


def is_zenith_cuda_available() -> bool:
    """True when libzenith_hip.so loads and a GPU is visible."""
    try:
        from .. import _lib

        _lib.load()
    except RuntimeError:
        return False
    return bool(torch.cuda.is_available())


# ------------------------------------------------------------ attention ---
def sdpa_pattern(q, k, v):
    """softmax(Q K^T / sqrt(d)) V written out (fx_patterns.py:81-92)."""
    scale = q.shape[-1] ** -0.5
    attn_weights = torch.matmul(q, k.transpose(-2, -1)) * scale
    attn_weights = F.softmax(attn_weights, dim=-1)
    return torch.matmul(attn_weights, v)


@torch.fx.wrap
def hip_flash_attention(q, k, v):
    """Leaf call into the HIP flash-attention kernel (scale 1/sqrt(head_dim),
    non-causal)."""
    return zenith_cuda.flash_attention(q, k, v)


def zenith_sdpa_replacement(q, k, v):
    return hip_flash_attention(q, k, v)


def sdpa_call_pattern(q, k, v):
    """The functional form F.scaled_dot_product_attention(q, k, v) with no
    mask, no dropout and is_causal=False (what torch's own BERT attention
    emits)."""
    return F.scaled_dot_product_attention(q, k, v)


# ----------------------------------------------------------- activation ---
def gelu_tanh_pattern(x):
    """0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3))) written out
    (fx_patterns.py:138-149)."""
    return 0.5 * x * (1.0 + torch.tanh(0.7978845608028654 * (x + 0.044715 * torch.pow(x, 3))))


@torch.fx.wrap
def hip_gelu_tanh(x):
    """Leaf call into the HIP tanh-GELU (the reference `zenith_cuda.gelu`)."""
    return zenith_cuda.gelu(x, approximate="tanh")


def zenith_gelu_replacement(x):
    return hip_gelu_tanh(x)


def gelu_erf_pattern(x):
    """Exact GELU through torch (F.gelu default, BERT hidden_act='gelu')."""
    return F.gelu(x)


@torch.fx.wrap
def hip_gelu_erf(x):
    return zenith_cuda.gelu(x, approximate="none")


def zenith_gelu_erf_replacement(x):
    return hip_gelu_erf(x)


def linear_gelu_pattern(x, w, b):
    """GELU(x W^T + b): the FFN-up Linear+GELU (GraphIR LinearGelu,
    zenith/optimization/fusion_pass.py:286-294)."""
    return F.gelu(F.linear(x, w, b))


@torch.fx.wrap
def hip_linear_gelu(x, w, b):
    """One MFMA GEMM with the bias + erf-GELU epilogue fused."""
    return zenith_cuda.linear(x, w, b, activation="gelu")


def zenith_linear_gelu_replacement(x, w, b):
    return hip_linear_gelu(x, w, b)


# -------------------------------------------------------- normalisation ---
def layernorm_pattern(x, weight, bias, eps=1e-5):
    """(x - mean) / sqrt(var + eps) * weight + bias written out
    (fx_patterns.py:163-173)."""
    mean = x.mean(dim=-1, keepdim=True)
    var = x.var(dim=-1, keepdim=True, unbiased=False)
    normalized = (x - mean) / torch.sqrt(var + eps)
    return normalized * weight + bias


def _rows(x):
    return x.reshape(-1, x.shape[-1])


@torch.fx.wrap
def hip_layernorm(x, weight, bias, eps=1e-5):
    """HIP LayerNorm over the last dimension of any-rank input."""
    return zenith_cuda.layernorm(_rows(x), weight, bias, eps).view(x.shape)


def zenith_layernorm_replacement(x, weight, bias, eps=1e-5):
    return hip_layernorm(x, weight, bias, eps)


def add_layernorm_pattern(x, residual, weight, bias):
    """LayerNorm(x + residual) via F.layer_norm, eps 1e-12 (BERT post-LN,
    GraphIR AddLayerNorm, fusion_pass.py:304-312)."""
    return F.layer_norm(x + residual, (x.shape[-1],), weight, bias, 1e-12)


@torch.fx.wrap
def hip_add_layernorm(x, residual, weight, bias):
    return zenith_cuda.add_layernorm(_rows(x), _rows(residual), weight, bias, 1e-12).view(x.shape)


def zenith_add_layernorm_replacement(x, residual, weight, bias):
    return hip_add_layernorm(x, residual, weight, bias)


# Leaves used by the optimizer's structural pass (module and functional
# forms with explicit eps / scale).
@torch.fx.wrap
def hip_add_layernorm_eps(x, residual, weight, bias, eps):
    """LayerNorm(x + residual) over the last dimension; a residual that
    broadcasts to x (a [1, S, H] position term, say) is expanded first."""
    if residual.shape != x.shape:
        residual = residual.expand(x.shape)
    return zenith_cuda.add_layernorm(_rows(x), _rows(residual), weight, bias, eps).view(x.shape)


@torch.fx.wrap
def hip_linear(x, w, b):
    return zenith_cuda.linear(x, w, b)


@torch.fx.wrap
def hip_attention(q, k, v, scale, attn_mask=None):
    return zenith_cuda.flash_attention(q, k, v, scale=scale, attn_mask=attn_mask)


# ------------------------------------------------------------- registry ---
def get_attention_patterns() -> list[FXPattern]:
    return [
        FXPattern("sdpa_to_flash", sdpa_pattern, zenith_sdpa_replacement, priority=20),
        FXPattern("sdpa_call_to_flash", sdpa_call_pattern, zenith_sdpa_replacement, priority=20),
    ]


def get_activation_patterns() -> list[FXPattern]:
    return [
        FXPattern("linear_gelu_to_epilogue", linear_gelu_pattern,
                  zenith_linear_gelu_replacement, priority=15),
        FXPattern("gelu_tanh_to_native", gelu_tanh_pattern, zenith_gelu_replacement, priority=10),
        FXPattern("gelu_erf_to_native", gelu_erf_pattern, zenith_gelu_erf_replacement, priority=10),
    ]


def get_normalization_patterns() -> list[FXPattern]:
    return [
        FXPattern("add_layernorm_to_fused", add_layernorm_pattern,
                  zenith_add_layernorm_replacement, priority=15),
        FXPattern("manual_layernorm_to_native", layernorm_pattern,
                  zenith_layernorm_replacement, priority=10),
    ]


def get_all_patterns() -> list[FXPattern]:
    return get_attention_patterns() + get_activation_patterns() + get_normalization_patterns()


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)

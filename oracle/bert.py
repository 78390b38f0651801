"""CPU oracle: BERT encoder layer composition. TEST INFRASTRUCTURE ONLY.

Post-LN layer in the order of the reference's GPU-resident encoder
(benchmarks/bert_fp16_full.py:96-145, bert_hybrid.py:96-146):
QKV projection -> split heads -> attention -> merge -> output projection
-> Add+LayerNorm -> FFN up + GELU -> FFN down -> Add+LayerNorm.
GELU is the exact erf form and eps 1e-12 for the workload configs (HF BERT
defaults; the reference scripts use gelu_new / 1e-5, bert_encoder.py:246-252).
"""

from __future__ import annotations

import numpy as np

from . import ops

F32 = np.float32


def _split(t: np.ndarray, B: int, S: int, heads: int) -> np.ndarray:
    H = t.shape[-1]
    return t.reshape(B, S, heads, H // heads).transpose(0, 2, 1, 3)


def bert_layer(x: np.ndarray, w: dict, lens: np.ndarray | None = None, heads: int = 12,
               eps: float = 1e-12, gelu: str = "erf", int8: dict | None = None,
               act_f16: bool = False, taps: dict | None = None) -> np.ndarray:
    """x [B, S, H] float32 -> [B, S, H]. `int8`, if given, holds the INT8-FFN
    operands {Wi_q, s_wi, Wo2_q, s_wo2, s_x, s_h} and replaces the two FFN
    GEMMs by quantised ones (int32 accumulate, dequant + bias + GELU, then
    dequant + bias before the residual Add+LayerNorm).

    act_f16=True models a pipeline that stores every tensor passed between
    kernels in fp16 (fp32 arithmetic inside each op): each such tensor is
    rounded to fp16. With int8=None and act_f16=False this is the plain fp32
    reference path.

    taps, if given, receives the FFN input h1 [B*S, H] and the GELU output
    u [B*S, FFN] (before any int8 quantisation): the activations whose
    absmax calibrates the INT8 FFN's two activation scales."""
    B, S, H = x.shape
    st = (lambda t: t.astype(np.float16).astype(F32)) if act_f16 else (lambda t: t)
    x2 = st(x.reshape(B * S, H).astype(F32))
    q = st(ops.linear(x2, w["Wq"], w["bq"]))
    k = st(ops.linear(x2, w["Wk"], w["bk"]))
    v = st(ops.linear(x2, w["Wv"], w["bv"]))
    ctx = ops.attention(_split(q, B, S, heads), _split(k, B, S, heads), _split(v, B, S, heads),
                        lens).astype(F32)
    ctx = st(ctx.transpose(0, 2, 1, 3).reshape(B * S, H))
    a = st(ops.linear(ctx, w["Wo"], w["bo"]))
    h1 = st(ops.add_layernorm(a, x2, w["ln1_g"], w["ln1_b"], eps))
    if int8 is None:
        u = st(ops.bias_gelu(ops.linear(h1, w["Wi"]), w["bi"], "tanh" if gelu == "tanh" else "erf"))
        d = st(ops.linear(u, w["Wo2"], w["bo2"]))
    else:
        act = "gelu_tanh" if gelu == "tanh" else "gelu"
        qh = ops.quantize_int8(h1, int8["s_x"])
        u = st(ops.int8_linear(qh, int8["Wi_q"], int8["s_x"], int8["s_wi"], w["bi"], act))
        qu = ops.quantize_int8(u, int8["s_h"])
        d = st(ops.int8_linear(qu, int8["Wo2_q"], int8["s_h"], int8["s_wo2"], w["bo2"]))
    if taps is not None:
        taps["h1"], taps["u"] = h1, u
    out = st(ops.add_layernorm(d, h1, w["ln2_g"], w["ln2_b"], eps))
    return out.reshape(B, S, H)


def bert_encoder(x: np.ndarray, layers: list[dict], lens: np.ndarray | None = None,
                 heads: int = 12, eps: float = 1e-12, gelu: str = "erf",
                 int8_layers: list[dict] | None = None, act_f16: bool = False) -> np.ndarray:
    h = x.astype(F32)
    for i, w in enumerate(layers):
        h = bert_layer(h, w, lens, heads, eps, gelu, None if int8_layers is None else int8_layers[i],
                       act_f16)
    return h


def ffn_activations(h1: np.ndarray, w: dict, gelu: str = "erf") -> np.ndarray:
    """GELU(h1 . Wi^T + bi): the FFN-up output whose absmax calibrates the
    second INT8 GEMM's activation scale."""
    return ops.bias_gelu(ops.linear(h1, w["Wi"]), w["bi"], "tanh" if gelu == "tanh" else "erf")

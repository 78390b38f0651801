"""The reference's GPU-resident "hybrid" BERT encoder, written against
zenith_amd.core_cuda (the ``_zenith_core.cuda`` API over the HIP kernels).

Same composition as benchmarks/bert_hybrid.py:96-146 (BertLayerHybrid) and
:149-168 (BertEncoderHybrid): fp32 Q/K/V/output/FFN linears, head split,
fp16 attention, head merge, fused Add+LayerNorm (eps 1e-5, the reference
call's default), tanh GELU (the benchmark builds its torch model with
hidden_act="gelu_new"), fused Add+LayerNorm. It is the workload of the
reference's published BERT comparator (b=1, s=128, 12 layers; 9.74 ms on a
T4, BENCHMARK_REPORT.md:54).
"""

from __future__ import annotations

import numpy as np

from . import core_cuda as cuda


def _np(t) -> np.ndarray:
    return t.detach().cpu().numpy().astype(np.float32)


class BertLayerHybrid:
    """One post-LN encoder layer; weights in torch-Linear layout W[out, in]."""

    def __init__(self, hidden_size: int = 768, num_heads: int = 12,
                 intermediate_size: int = 3072, eps: float = 1e-5):
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.head_dim = hidden_size // num_heads
        self.intermediate_size = intermediate_size
        self.eps = eps
        self.w: dict[str, cuda.GpuTensor] = {}

    def load_weights(self, w: dict) -> "BertLayerHybrid":
        """From a dict of numpy arrays with the keys Wq, bq, Wk, bk, Wv, bv,
        Wo, bo, ln1_g, ln1_b, Wi, bi, Wo2, bo2, ln2_g, ln2_b."""
        self.w = {k: cuda.to_gpu(np.asarray(v, np.float32)) for k, v in w.items()}
        return self

    def load_from_pytorch(self, torch_layer) -> "BertLayerHybrid":
        """From a transformers BertLayer (bert_hybrid.py:45-94)."""
        a, o = torch_layer.attention, torch_layer.output
        return self.load_weights({
            "Wq": _np(a.self.query.weight), "bq": _np(a.self.query.bias),
            "Wk": _np(a.self.key.weight), "bk": _np(a.self.key.bias),
            "Wv": _np(a.self.value.weight), "bv": _np(a.self.value.bias),
            "Wo": _np(a.output.dense.weight), "bo": _np(a.output.dense.bias),
            "ln1_g": _np(a.output.LayerNorm.weight), "ln1_b": _np(a.output.LayerNorm.bias),
            "Wi": _np(torch_layer.intermediate.dense.weight),
            "bi": _np(torch_layer.intermediate.dense.bias),
            "Wo2": _np(o.dense.weight), "bo2": _np(o.dense.bias),
            "ln2_g": _np(o.LayerNorm.weight), "ln2_b": _np(o.LayerNorm.bias),
        })

    def forward(self, x_gpu: cuda.GpuTensor, batch_size: int, seq_len: int) -> cuda.GpuTensor:
        w, nh, hd = self.w, self.num_heads, self.head_dim
        q = cuda.linear_gpu(x_gpu, w["Wq"], w["bq"])
        k = cuda.linear_gpu(x_gpu, w["Wk"], w["bk"])
        v = cuda.linear_gpu(x_gpu, w["Wv"], w["bv"])
        q4 = cuda.transpose_for_attention(q, batch_size, seq_len, nh, hd)
        k4 = cuda.transpose_for_attention(k, batch_size, seq_len, nh, hd)
        v4 = cuda.transpose_for_attention(v, batch_size, seq_len, nh, hd)
        ctx = cuda.attention_fp16_gpu(q4, k4, v4)
        ctx4 = cuda.transpose_from_attention(ctx, batch_size, nh, seq_len, hd)
        ctx2 = cuda.reshape_4d_to_2d(ctx4, batch_size, seq_len, self.hidden_size)
        proj = cuda.linear_gpu(ctx2, w["Wo"], w["bo"])
        hidden = cuda.fused_add_layernorm_gpu(proj, x_gpu, w["ln1_g"], w["ln1_b"], self.eps)
        up = cuda.gelu_gpu(cuda.linear_gpu(hidden, w["Wi"], w["bi"]))
        down = cuda.linear_gpu(up, w["Wo2"], w["bo2"])
        return cuda.fused_add_layernorm_gpu(down, hidden, w["ln2_g"], w["ln2_b"], self.eps)


class BertEncoderHybrid:
    """A stack of BertLayerHybrid (bert_hybrid.py:149-168)."""

    def __init__(self, num_layers: int = 12, hidden_size: int = 768, num_heads: int = 12,
                 intermediate_size: int = 3072, eps: float = 1e-5):
        self.layers = [BertLayerHybrid(hidden_size, num_heads, intermediate_size, eps)
                       for _ in range(num_layers)]

    def load_weights(self, layers: list[dict]) -> "BertEncoderHybrid":
        for layer, w in zip(self.layers, layers, strict=True):
            layer.load_weights(w)
        return self

    def load_from_pytorch(self, torch_encoder) -> "BertEncoderHybrid":
        for layer, tl in zip(self.layers, torch_encoder.layer, strict=True):
            layer.load_from_pytorch(tl)
        return self

    def forward(self, x_gpu: cuda.GpuTensor, batch_size: int, seq_len: int) -> cuda.GpuTensor:
        hidden = x_gpu
        for layer in self.layers:
            hidden = layer.forward(hidden, batch_size, seq_len)
        return hidden

"""BERT from input_ids on the HIP kernels: the fused embedding layer
(zk_bert_embeddings) in front of the fp16 encoder (zenith_amd.encoder), and
a weight loader for Hugging Face BERT checkpoints.

The loader takes a transformers BertModel (or a model that holds one as
`.bert`), a state dict, or a checkpoint directory (config.json plus
model.safetensors, or pytorch_model.bin read with weights_only=True); HF
stores Linear weights as W[out, in], which is the layout the encoder keeps
(the reference's load_from_pytorch, benchmarks/bert_fp16_full.py:45-94, and
bert_hybrid.py:45-94, read the same tensors). hidden_act "gelu" selects the
erf GELU epilogue and "gelu_new" / "gelu_pytorch_tanh" the tanh one.

`forward` returns last_hidden_state; `pool` is the pooler head,
tanh(dense(h[:, 0])) over the [CLS] rows (the reference's BERT benchmark
model, benchmarks/bert_benchmark.py:101-107, and transformers' BertPooler),
present when the checkpoint holds pooler weights.
"""

from __future__ import annotations

import json
import os

import numpy as np
import torch

from . import _lib as L
from .encoder import BertEncoder
from .zenith_cuda import _ws_args, gemm_workspace

F16 = torch.float16

_LAYER_KEYS = {
    "Wq": "attention.self.query.weight", "bq": "attention.self.query.bias",
    "Wk": "attention.self.key.weight", "bk": "attention.self.key.bias",
    "Wv": "attention.self.value.weight", "bv": "attention.self.value.bias",
    "Wo": "attention.output.dense.weight", "bo": "attention.output.dense.bias",
    "ln1_g": "attention.output.LayerNorm.weight", "ln1_b": "attention.output.LayerNorm.bias",
    "Wi": "intermediate.dense.weight", "bi": "intermediate.dense.bias",
    "Wo2": "output.dense.weight", "bo2": "output.dense.bias",
    "ln2_g": "output.LayerNorm.weight", "ln2_b": "output.LayerNorm.bias",
}
_EMB_KEYS = {
    "word": "embeddings.word_embeddings.weight",
    "pos": "embeddings.position_embeddings.weight",
    "type": "embeddings.token_type_embeddings.weight",
    "ln_g": "embeddings.LayerNorm.weight", "ln_b": "embeddings.LayerNorm.bias",
}
_POOLER_KEYS = {"W": "pooler.dense.weight", "b": "pooler.dense.bias"}
_GELU = {"gelu": "erf", "gelu_new": "tanh", "gelu_pytorch_tanh": "tanh", "gelu_fast": "tanh"}


def _np32(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        t = t.detach().to(torch.float32).cpu().numpy()
    return np.ascontiguousarray(np.asarray(t, dtype=np.float32))


def split_state_dict(sd: dict, num_layers: int) -> tuple[dict, list[dict]]:
    """HF BERT state dict (with or without a leading "bert.") -> (embedding
    tables, per-layer weight dicts in the encoder's key names)."""
    prefix = _prefix(sd)
    get = lambda k: _np32(sd[prefix + k])  # noqa: E731
    emb = {n: get(k) for n, k in _EMB_KEYS.items()}
    layers = [{n: get(f"encoder.layer.{i}.{k}") for n, k in _LAYER_KEYS.items()}
              for i in range(num_layers)]
    return emb, layers


def pooler_weights(sd: dict) -> dict | None:
    """{"W": [H, H], "b": [H]} of the pooler dense layer, or None when the
    state dict has none (add_pooling_layer=False, masked-LM heads)."""
    prefix = _prefix(sd)
    if prefix + _POOLER_KEYS["W"] not in sd:
        return None
    return {n: _np32(sd[prefix + k]) for n, k in _POOLER_KEYS.items()}


def _prefix(sd: dict) -> str:
    return "bert." if any(k.startswith("bert.") for k in sd) else ""


class BertModel:
    """Embeddings + encoder; input_ids [B, S] -> last_hidden_state [B, S, H] fp16."""

    def __init__(self, emb: dict, layers: list[dict], heads: int = 12, eps: float = 1e-12,
                 gelu: str = "erf", device: str | torch.device = "cuda",
                 pooler: dict | None = None):
        self.device = torch.device(device)
        L.load()
        self.eps = float(eps)
        self.encoder = BertEncoder(layers, heads=heads, eps=eps, gelu=gelu, device=self.device)
        to = lambda a: torch.from_numpy(_np32(a)).to(self.device, F16).contiguous()  # noqa: E731
        self.word, self.pos, self.type = to(emb["word"]), to(emb["pos"]), to(emb["type"])
        self.ln_g, self.ln_b = to(emb["ln_g"]), to(emb["ln_b"])
        self.hidden = self.word.shape[1]
        self.pool_w = self.pool_b = None
        if pooler is not None:
            self.pool_w, self.pool_b = to(pooler["W"]), to(pooler["b"])
            if self.pool_w.shape != (self.hidden, self.hidden) or self.pool_b.shape != (self.hidden,):
                raise RuntimeError("pooler weights must be [hidden, hidden] and [hidden]")

    # ----------------------------------------------------------- loaders --
    @classmethod
    def from_hf(cls, model, device: str | torch.device = "cuda") -> "BertModel":
        """From a transformers BertModel (or a model with a `.bert` member)."""
        bert = getattr(model, "bert", model)
        cfg = bert.config
        sd = bert.state_dict()
        emb, layers = split_state_dict(sd, cfg.num_hidden_layers)
        return cls(emb, layers, heads=cfg.num_attention_heads, eps=cfg.layer_norm_eps,
                   gelu=_GELU.get(cfg.hidden_act, "erf"), device=device,
                   pooler=pooler_weights(sd))

    @classmethod
    def from_pretrained(cls, path: str, device: str | torch.device = "cuda") -> "BertModel":
        """From a checkpoint directory: config.json and model.safetensors
        (or pytorch_model.bin, loaded with weights_only=True)."""
        with open(os.path.join(path, "config.json")) as f:
            cfg = json.load(f)
        st = os.path.join(path, "model.safetensors")
        if os.path.exists(st):
            from safetensors.numpy import load_file

            sd = load_file(st)
        else:
            sd = torch.load(os.path.join(path, "pytorch_model.bin"), map_location="cpu",
                            weights_only=True)
        emb, layers = split_state_dict(sd, int(cfg["num_hidden_layers"]))
        return cls(emb, layers, heads=int(cfg["num_attention_heads"]),
                   eps=float(cfg.get("layer_norm_eps", 1e-12)),
                   gelu=_GELU.get(cfg.get("hidden_act", "gelu"), "erf"), device=device,
                   pooler=pooler_weights(sd))

    # ----------------------------------------------------------- forward --
    def embed(self, input_ids: torch.Tensor, token_type_ids: torch.Tensor | None = None,
              pos_offset: int = 0) -> torch.Tensor:
        """input_ids [B, S] -> LayerNorm(word + position + token type) fp16."""
        ids = self._ids(input_ids)
        tt = None if token_type_ids is None else self._ids(token_type_ids)
        if tt is not None and tt.shape != ids.shape:
            raise RuntimeError("token_type_ids must match input_ids")
        B, S = ids.shape
        out = torch.empty((B, S, self.hidden), dtype=F16, device=self.device)
        L.call("zk_bert_embeddings", ids.data_ptr(), None if tt is None else tt.data_ptr(),
               self.word.data_ptr(), self.pos.data_ptr(), self.type.data_ptr(),
               self.ln_g.data_ptr(), self.ln_b.data_ptr(), out.data_ptr(), B, S, self.hidden,
               self.word.shape[0], self.pos.shape[0], self.type.shape[0], int(pos_offset),
               self.eps, L.ZK_F16, torch.cuda.current_stream(self.device).cuda_stream)
        return out

    def forward(self, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None,
                token_type_ids: torch.Tensor | None = None,
                lengths: torch.Tensor | None = None) -> torch.Tensor:
        """last_hidden_state [B, S, H] fp16. Padding is given either as
        per-sequence `lengths` (int32 [B]) or as a right-padded 0/1
        `attention_mask` [B, S]."""
        x = self.embed(input_ids, token_type_ids)
        if lengths is None and attention_mask is not None:
            lengths = self._mask_to_lengths(attention_mask, x.shape[1])
        return self.encoder(x, lengths)

    __call__ = forward

    def pool(self, hidden: torch.Tensor) -> torch.Tensor:
        """pooler_output [B, H] fp16 = tanh(hidden[:, 0] @ W^T + b). The
        GEMM reads the [CLS] rows in place (leading dimension S*H) with the
        bias in its epilogue; tanh runs in place on the [B, H] result."""
        if self.pool_w is None:
            raise RuntimeError("this model has no pooler weights")
        if (hidden.dim() != 3 or hidden.shape[2] != self.hidden or hidden.dtype != F16
                or not hidden.is_contiguous() or hidden.device.type != "cuda"):
            raise RuntimeError("pool expects the contiguous fp16 [B, S, hidden] encoder output")
        B, S, H = hidden.shape
        out = torch.empty((B, H), dtype=F16, device=self.device)
        if B == 0:
            return out
        stream = torch.cuda.current_stream(self.device).cuda_stream
        ws = gemm_workspace(B, H, H, L.ZK_F16, self.device)
        L.call("zk_gemm_f16_ws", hidden.data_ptr(), self.pool_w.data_ptr(), out.data_ptr(),
               B, H, H, S * H, H, H, 1, L.ZK_F16, self.pool_b.data_ptr(), None, 0, L.ZK_EPI_BIAS,
               *_ws_args(ws), stream)
        L.call("zk_tanh", out.data_ptr(), out.data_ptr(), B * H, L.ZK_F16, stream)
        return out

    def _ids(self, t) -> torch.Tensor:
        t = torch.as_tensor(t)
        if t.dim() != 2:
            raise RuntimeError("ids must be [batch, seq]")
        return t.to(device=self.device, dtype=torch.int32).contiguous()

    def _mask_to_lengths(self, mask, S: int) -> torch.Tensor:
        m = torch.as_tensor(mask).to(self.device)
        if m.dim() != 2 or m.shape[1] != S:
            raise RuntimeError("attention_mask must be [batch, seq]")
        lens = (m != 0).sum(dim=1, dtype=torch.int32)
        prefix = torch.arange(S, device=self.device)[None, :] < lens[:, None]
        if not torch.equal(prefix, m != 0):
            raise RuntimeError("attention_mask must be a right-padded prefix mask (1s then 0s)")
        return lens.contiguous()

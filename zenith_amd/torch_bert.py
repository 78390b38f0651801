"""A plain PyTorch post-LN BERT layer (nn.Linear / nn.LayerNorm / nn.GELU /
F.scaled_dot_product_attention) in the layer order of the reference's
encoder scripts (benchmarks/bert_fp16_full.py:96-145). It is the model the
graph hooks are applied to: FX rewriting or torch.compile with the zenith
backend turns its modules into the HIP kernels. Weights come from the same
dicts the encoder and the oracle use (torch-Linear layout W[out, in])."""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn


class TorchBertLayer(nn.Module):
    def __init__(self, w: dict, heads: int = 12, eps: float = 1e-12):
        super().__init__()
        H, I = w["Wq"].shape[1], w["Wi"].shape[0]
        self.heads = heads
        self.q, self.k, self.v, self.o = (nn.Linear(H, H) for _ in range(4))
        self.ln1 = nn.LayerNorm(H, eps=eps)
        self.i = nn.Linear(H, I)
        self.act = nn.GELU()
        self.o2 = nn.Linear(I, H)
        self.ln2 = nn.LayerNorm(H, eps=eps)
        pairs = [(self.q, "Wq", "bq"), (self.k, "Wk", "bk"), (self.v, "Wv", "bv"),
                 (self.o, "Wo", "bo"), (self.i, "Wi", "bi"), (self.o2, "Wo2", "bo2"),
                 (self.ln1, "ln1_g", "ln1_b"), (self.ln2, "ln2_g", "ln2_b")]
        with torch.no_grad():
            for mod, wk, bk in pairs:
                mod.weight.copy_(torch.as_tensor(w[wk]))
                mod.bias.copy_(torch.as_tensor(w[bk]))

    def _split(self, t, B, S):
        return t.view(B, S, self.heads, -1).transpose(1, 2)

    def _rest(self, a, x):
        B, S, H = x.shape
        a = a.transpose(1, 2).reshape(B, S, H)
        h = self.ln1(self.o(a) + x)
        return self.ln2(self.o2(self.act(self.i(h))) + h)

    def forward(self, x):
        B, S, _ = x.shape
        sp = lambda t: self._split(t, B, S)  # noqa: E731
        return self._rest(F.scaled_dot_product_attention(sp(self.q(x)), sp(self.k(x)),
                                                         sp(self.v(x))), x)


class MaskedTorchBertLayer(TorchBertLayer):
    """TorchBertLayer over a padded batch: forward(x, attn_mask) with the
    boolean [B, 1, S, S] mask (True = attend) that HF BERT's SDPA attention
    passes."""

    def forward(self, x, attn_mask):
        B, S, _ = x.shape
        sp = lambda t: self._split(t, B, S)  # noqa: E731
        return self._rest(F.scaled_dot_product_attention(sp(self.q(x)), sp(self.k(x)),
                                                         sp(self.v(x)), attn_mask=attn_mask), x)

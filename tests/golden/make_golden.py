"""Writes the committed golden fixtures under tests/golden/.

config1_bert_layer.npz: config 1 (one post-LN BERT layer, b1 s128, hidden 768,
12 heads, FFN 3072, erf GELU, eps 1e-12, weights ~N(0,0.02) seed 42, x ~N(0,1))
evaluated by transformers.BertLayer (torch CPU fp32, eager attention) - an
implementation independent of this repository's oracle. Stores the output
`y` and a corner of the seeded input to detect generator drift.

Run: python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests.test_oracle import _hf_layer  # noqa: E402
from zenith_amd import synthetic  # noqa: E402


def main():
    w = synthetic.bert_weights(1, seed=42)[0]
    x = synthetic.hidden_states(1, 128, seed=42)
    layer = _hf_layer(w, eps=1e-12)
    with torch.no_grad():
        out = layer(torch.from_numpy(x))
    y = (out[0] if isinstance(out, tuple) else out).numpy().astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "config1_bert_layer.npz"), y=y, x_corner=x[0, :4, :4])
    print("wrote config1_bert_layer.npz", y.shape, float(np.abs(y).max()))


if __name__ == "__main__":
    main()

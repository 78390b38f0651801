"""Seeded synthetic inputs for the BERT-encoder workloads.

No datasets or checkpoints are available offline, so every benchmark and
parity test draws its inputs here, from numpy's PCG64 (`default_rng`) with the
reference's seed 42 (tests/python/test_numerical_accuracy.py:47,
benchmarks/bert_encoder.py:320). Distributions follow the workload configs:
weights ~ N(0, 0.02), biases 0, LayerNorm gamma 1 / beta 0, activations
~ N(0, 1), key-padding lengths ~ U{S/2 .. S}.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32

LAYER_KEYS = ("Wq", "bq", "Wk", "bk", "Wv", "bv", "Wo", "bo", "ln1_g", "ln1_b",
              "Wi", "bi", "Wo2", "bo2", "ln2_g", "ln2_b")


def bert_layer_weights(rng: np.random.Generator, hidden: int = 768, ffn: int = 3072,
                       std: float = 0.02) -> dict[str, np.ndarray]:
    """One post-LN BERT layer in torch-Linear layout (W[out, in])."""

    def w(o, i):
        return (rng.standard_normal((o, i), dtype=F32) * F32(std)).astype(F32)

    H, I = hidden, ffn
    return {
        "Wq": w(H, H), "bq": np.zeros(H, F32),
        "Wk": w(H, H), "bk": np.zeros(H, F32),
        "Wv": w(H, H), "bv": np.zeros(H, F32),
        "Wo": w(H, H), "bo": np.zeros(H, F32),
        "ln1_g": np.ones(H, F32), "ln1_b": np.zeros(H, F32),
        "Wi": w(I, H), "bi": np.zeros(I, F32),
        "Wo2": w(H, I), "bo2": np.zeros(H, F32),
        "ln2_g": np.ones(H, F32), "ln2_b": np.zeros(H, F32),
    }


def bert_weights(num_layers: int = 12, hidden: int = 768, ffn: int = 3072,
                 seed: int = 42) -> list[dict[str, np.ndarray]]:
    rng = np.random.default_rng(seed)
    return [bert_layer_weights(rng, hidden, ffn) for _ in range(num_layers)]


def perturb_norms_and_biases(layers: list[dict[str, np.ndarray]], seed: int = 42,
                             g_std: float = 0.1, b_std: float = 0.1, bias_std: float = 0.05,
                             q_bias_std: float = 0.5) -> list[dict[str, np.ndarray]]:
    """Copies of `layers` with every LayerNorm gamma ~ 1 + N(0, g_std), beta
    ~ N(0, b_std), the query bias ~ N(0, q_bias_std) and every other Linear
    bias ~ N(0, bias_std), drawn per layer, so that no two layers share a
    LayerNorm and no bias is zero (a trained checkpoint's situation). The
    matrices are kept. Wiring mistakes that the default weights (gamma 1,
    beta 0, biases 0 in every layer) cannot show, such as one layer's
    LayerNorm applied in another layer, a dropped bias or beta term, or
    Q/K/V biases interleaved differently from their weights, change the
    output under these weights. The query bias is the larger one because a
    key bias adds the same amount to every logit of a query and cancels in
    the softmax: a query/key bias swap shows only through the query bias's
    own effect on the logits, q_bias . k / sqrt(D)."""
    rng = np.random.default_rng([seed, 3])
    out = []
    for w in layers:
        w = dict(w)
        for k in ("ln1_g", "ln2_g"):
            w[k] = (1.0 + rng.standard_normal(w[k].shape) * g_std).astype(F32)
        for k in ("ln1_b", "ln2_b"):
            w[k] = (rng.standard_normal(w[k].shape) * b_std).astype(F32)
        for k in ("bq", "bk", "bv", "bo", "bi", "bo2"):
            std = q_bias_std if k == "bq" else bias_std
            w[k] = (rng.standard_normal(w[k].shape) * std).astype(F32)
        out.append(w)
    return out


def bert_weights_wired(num_layers: int = 12, hidden: int = 768, ffn: int = 3072,
                       seed: int = 42) -> list[dict[str, np.ndarray]]:
    """bert_weights with per-layer LayerNorm parameters and non-zero biases
    (perturb_norms_and_biases): the weight set of the composition tests."""
    return perturb_norms_and_biases(bert_weights(num_layers, hidden, ffn, seed), seed)


def hidden_states(batch: int, seq: int, hidden: int = 768, seed: int = 42) -> np.ndarray:
    """Token embeddings ~ N(0, 1), [batch, seq, hidden] float32."""
    rng = np.random.default_rng([seed, 1])
    return rng.standard_normal((batch, seq, hidden), dtype=F32)


def padding_lengths(batch: int, seq: int, seed: int = 42) -> np.ndarray:
    """Per-sequence valid lengths ~ U{seq/2 .. seq} (inclusive), int32."""
    rng = np.random.default_rng([seed, 2])
    return rng.integers(seq // 2, seq, size=batch, endpoint=True).astype(np.int32)


def uniform(shape, seed: int = 42, tag: int = 0, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    rng = np.random.default_rng([seed, 100 + tag])
    return rng.uniform(lo, hi, size=shape).astype(F32)


def normal(shape, seed: int = 42, tag: int = 0, std: float = 1.0) -> np.ndarray:
    rng = np.random.default_rng([seed, 200 + tag])
    return (rng.standard_normal(shape, dtype=F32) * F32(std)).astype(F32)


def round_f16(a: np.ndarray) -> np.ndarray:
    """The float32 image of a's float16 rounding (what an fp16 kernel sees)."""
    return a.astype(np.float16).astype(F32)

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

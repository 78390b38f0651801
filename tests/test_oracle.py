"""Pins for the CPU oracle (oracle/). Each oracle function is checked against
something independent of its own formula:

  matmul / linear      reference KAT (tests/test_kernels.cpp:68-86); the
                       reference's own cpu_kernels.cpp built into oracle/_ref;
                       own AVX2 restatement vs reference build (same loop)
  softmax              reference softmax_f32 (oracle/_ref)
  layernorm/add_ln     reference fused.add_layernorm (oracle/_ref,
                       features_bindings.hpp); torch.nn.functional.layer_norm;
                       unit mean/std invariant
  gelu_tanh / erf      reference fused.bias_gelu (oracle/_ref); reference KATs
                       (tests/test_cuda_cublas_bindings.py:36-57); torch F.gelu
  attention            torch SDPA with a boolean key mask; closed forms
                       (Sk=1 -> V, uniform keys -> mean(V), all-masked -> 0)
  quantize/int8        int64 brute force, round-half-even / clamp cases,
                       |x - dq(q(x))| <= s/2 (tests/test_quantization.py:14-37)
  bert_layer           transformers.BertLayer random-init (hidden_act gelu,
                       eps 1e-12) with the same weights; committed golden of
                       config 1 made by that model (tests/golden/)
"""

import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import bert as obert
from oracle import native, ops
from zenith_amd import synthetic

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
needs_ref = pytest.mark.skipif(not native.ref_available(), reason="oracle/_ref not built")


# ------------------------------------------------------------------ GEMM ---
def test_matmul_reference_kat():
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[1, 2], [3, 4], [5, 6]], np.float32)
    np.testing.assert_array_equal(ops.matmul(a, b), [[22, 28], [49, 64]])
    np.testing.assert_array_equal(native.own_gemm().matmul(a, b), [[22, 28], [49, 64]])


def test_identity_and_zero_invariants():
    a = synthetic.uniform((17, 9), tag=1)
    np.testing.assert_array_equal(ops.matmul(a, np.eye(9, dtype=np.float32)), a)
    assert not ops.matmul(a, np.zeros((9, 4), np.float32)).any()


@needs_ref
@pytest.mark.parametrize("M,K,N", [(2, 3, 2), (33, 70, 19), (128, 768, 768)])
def test_matmul_vs_reference_build(M, K, N):
    a = synthetic.uniform((M, K), tag=2)
    b = synthetic.uniform((K, N), tag=3)
    ref = native.ref_gemm()
    r_avx = ref.matmul(a, b, "avx2")
    np.testing.assert_allclose(ops.matmul(a, b), r_avx, rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(ops.matmul(a, b), ref.matmul(a, b, "naive"), rtol=1e-5, atol=1e-4)
    # the own C restatement reproduces the reference loop exactly
    np.testing.assert_array_equal(native.own_gemm().matmul(a, b, "avx2"), r_avx)


def test_linear_layout():
    x = synthetic.normal((5, 8), tag=4)
    w = synthetic.normal((3, 8), tag=5)
    b = synthetic.normal((3,), tag=6)
    np.testing.assert_allclose(ops.linear(x, w, b), x @ w.T + b, rtol=1e-6, atol=1e-6)
    tl = F.linear(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b)).numpy()
    np.testing.assert_allclose(ops.linear(x, w, b), tl, rtol=1e-5, atol=1e-6)


# --------------------------------------------------------------- softmax ---
@needs_ref
def test_softmax_vs_reference_build():
    x = synthetic.normal((7, 130), tag=7) * 5
    np.testing.assert_allclose(ops.softmax(x), native.ref_softmax(x), rtol=1e-6, atol=1e-7)


# ----------------------------------------------------------------- norms ---
@pytest.mark.parametrize("eps", [1e-12, 1e-5])
def test_layernorm_vs_torch(eps):
    x = synthetic.normal((64, 768), tag=8) * 3 + 1
    g = synthetic.normal((768,), tag=9) + 1
    b = synthetic.normal((768,), tag=10)
    t = F.layer_norm(torch.from_numpy(x), (768,), torch.from_numpy(g), torch.from_numpy(b), eps).numpy()
    np.testing.assert_allclose(ops.layernorm(x, g, b, eps), t, rtol=1e-4, atol=1e-5)
    y = ops.layernorm(x, np.ones(768, np.float32), np.zeros(768, np.float32), eps)
    np.testing.assert_allclose(y.mean(-1), 0, atol=1e-5)
    np.testing.assert_allclose(y.std(-1), 1, atol=1e-4)


@needs_ref
def test_add_layernorm_vs_reference_build():
    mod = native.ref_features()
    x = synthetic.normal((32, 768), tag=11) * 2
    r = synthetic.normal((32, 768), tag=12)
    g = synthetic.normal((768,), tag=13) + 1
    b = synthetic.normal((768,), tag=14)
    for eps in (1e-12, 1e-5):
        np.testing.assert_allclose(ops.add_layernorm(x, r, g, b, eps),
                                   mod.fused.add_layernorm(x, r, g, b, eps), rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("eps", [1e-12, 1e-5])
def test_layernorm_add_vs_torch(eps):
    """LN(x) * g + b + r: torch's F.layer_norm plus the residual; with unit
    affine the residual-free part has unit-normal rows; and it differs from
    the pre-add LN(x + r) (a swapped residual placement fails here)."""
    x = synthetic.normal((64, 768), tag=15) * 2 + 0.5
    r = synthetic.normal((64, 768), tag=16)
    g = synthetic.normal((768,), tag=17) + 1
    b = synthetic.normal((768,), tag=18)
    t = (F.layer_norm(torch.from_numpy(x), (768,), torch.from_numpy(g), torch.from_numpy(b), eps)
         + torch.from_numpy(r)).numpy()
    y = ops.layernorm_add(x, r, g, b, eps)
    np.testing.assert_allclose(y, t, rtol=1e-4, atol=1e-5)
    one, zero = np.ones(768, np.float32), np.zeros(768, np.float32)
    y1 = ops.layernorm_add(x, r, one, zero, eps) - r
    np.testing.assert_allclose(y1.mean(-1), 0, atol=1e-5)
    np.testing.assert_allclose(y1.std(-1), 1, atol=1e-4)
    assert np.abs(y - ops.add_layernorm(x, r, g, b, eps)).max() > 0.5


# ------------------------------------------------------------------ GELU ---
def test_sigmoid_tanh_closed_forms():
    """sigmoid(0) = 1/2, sigmoid(x) + sigmoid(-x) = 1, saturation at +-inf,
    tanh(x) = 2 sigmoid(2x) - 1, and both vs torch's library routines."""
    import torch

    assert ops.sigmoid(np.zeros(3, np.float32)).tolist() == [0.5] * 3
    assert ops.sigmoid(np.array([-np.inf, np.inf], np.float32)).tolist() == [0.0, 1.0]
    x = np.linspace(-12, 12, 2001, dtype=np.float32)
    np.testing.assert_allclose(ops.sigmoid(x) + ops.sigmoid(-x), 1.0, atol=1e-6)
    np.testing.assert_allclose(ops.tanh(x), 2 * ops.sigmoid(2 * x) - 1, atol=2e-6)
    np.testing.assert_allclose(ops.tanh(-x), -ops.tanh(x), atol=0)
    t = torch.from_numpy(x)
    np.testing.assert_allclose(ops.sigmoid(x), torch.sigmoid(t).numpy(), rtol=2e-7, atol=1e-7)
    np.testing.assert_allclose(ops.tanh(x), torch.tanh(t).numpy(), rtol=2e-7, atol=1e-7)


def test_gelu_reference_kats():
    for fn in (ops.gelu_tanh, ops.gelu_erf):
        y = fn(np.array([1.0, 0.0, -1.0], np.float32))
        assert abs(y[0] - 0.841) < 0.01 and y[1] == 0 and abs(y[2] + 0.159) < 0.01


def test_gelu_vs_torch():
    x = synthetic.normal((10000,), tag=15) * 4
    tx = torch.from_numpy(x)
    np.testing.assert_allclose(ops.gelu_tanh(x), F.gelu(tx, approximate="tanh").numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ops.gelu_erf(x), F.gelu(tx).numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ops.gelu_tanh(x), ops.gelu_tanh_f64(x), rtol=1e-5, atol=1e-6)


@needs_ref
def test_bias_gelu_vs_reference_build():
    mod = native.ref_features()
    x = synthetic.normal((64, 3072), tag=16) * 3
    b = synthetic.normal((3072,), tag=17)
    np.testing.assert_allclose(ops.bias_gelu(x, b, "tanh"), mod.fused.bias_gelu(x, b), rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------- attention ---
def test_attention_vs_torch_sdpa_masked():
    B, H, S, D = 3, 2, 40, 64
    q, k, v = (synthetic.normal((B, H, S, D), tag=t) for t in (18, 19, 20))
    lens = np.array([40, 21, 1])
    mask = torch.from_numpy(np.arange(S)[None, :] < lens[:, None])[:, None, None, :]
    t = F.scaled_dot_product_attention(*(torch.from_numpy(a).double() for a in (q, k, v)), attn_mask=mask).numpy()
    np.testing.assert_allclose(ops.attention(q, k, v, lens), t, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(ops.attention(q, k, v), F.scaled_dot_product_attention(
        *(torch.from_numpy(a).double() for a in (q, k, v))).numpy(), rtol=1e-10, atol=1e-12)


def test_attention_general_mask_vs_torch_sdpa():
    """A boolean mask per (query, key) with rows that mask everything:
    torch SDPA's boolean attn_mask where at least one key is kept, and
    exactly 0 (the masked-primitive rule) for rows with none kept; a mask
    equal to the valid-length prefix matches valid_lens."""
    B, H, S, D = 2, 3, 24, 16
    q, k, v = (synthetic.normal((B, H, S, D), tag=t) for t in (24, 25, 26))
    rng = np.random.default_rng(5)
    mask = rng.random((B, 1, S, S)) < 0.6
    mask[0, 0, 3, :] = False  # a query with no key left
    o = ops.attention(q, k, v, mask=mask)
    t = F.scaled_dot_product_attention(*(torch.from_numpy(a).double() for a in (q, k, v)),
                                       attn_mask=torch.from_numpy(mask)).numpy()
    rows = mask.any(-1)  # [B,1,S]
    keep = np.broadcast_to(rows[..., None], o.shape)
    np.testing.assert_allclose(o[keep], t[keep], rtol=1e-10, atol=1e-12)
    assert not o[0, :, 3].any()
    lens = np.array([24, 9])
    prefix = (np.arange(S)[None, :] < lens[:, None])[:, None, None, :]
    np.testing.assert_allclose(ops.attention(q, k, v, mask=prefix), ops.attention(q, k, v, lens),
                               rtol=0, atol=0)


def test_attention_closed_forms():
    B, H, S, D = 2, 2, 16, 8
    q, k, v = (synthetic.normal((B, H, S, D), tag=t) for t in (21, 22, 23))
    # one key: output is that key's value row
    np.testing.assert_allclose(ops.attention(q, k[:, :, :1], v[:, :, :1]),
                               np.broadcast_to(v[:, :, :1], (B, H, S, D)), rtol=1e-12)
    # identical keys: uniform weights over the valid keys
    ku = np.broadcast_to(k[:, :, :1], k.shape)
    o = ops.attention(q, ku, v, np.array([5, 16]))
    np.testing.assert_allclose(o[0], np.broadcast_to(v[0, :, :5].astype(np.float64).mean(1, keepdims=True), o[0].shape), rtol=1e-10)
    # all keys masked: exactly zero (nan_to_num rule)
    assert not ops.attention(q, k, v, np.array([0, 3]))[0].any()
    # default scale is 1/sqrt(D)
    np.testing.assert_allclose(ops.attention(q, k, v), ops.attention(q, k, v, scale=1 / math.sqrt(D)))


# ------------------------------------------------------------------ int8 ---
def test_quantize_rounding_and_clamp():
    s = np.float32(0.5)
    x = np.array([0.25, 0.75, -0.25, -0.75, 1.25, 100, -100, 63.75, -64.25], np.float32)
    np.testing.assert_array_equal(ops.quantize_int8(x, s), [0, 2, 0, -2, 2, 127, -128, 127, -128])


def test_quantize_non_finite_matches_reference_rule():
    """Non-finite inputs: the reference's numpy rule (benchmarks/int8_bench.py:
    24, np.clip(np.round(x / scale), -128, 127).astype(np.int8)) as it runs
    on this host gives 0 for NaN and saturates the infinities; the oracle
    gives the same without relying on the platform-defined NaN cast."""
    s = np.float32(0.04)
    x = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 1.0, -1.0], np.float32)
    with np.errstate(invalid="ignore"):
        rule = np.clip(np.round(x / s), -128, 127).astype(np.int8)
    np.testing.assert_array_equal(rule, [0, 0, 127, -128, 0, 0, 25, -25])
    np.testing.assert_array_equal(ops.quantize_int8(x, s), rule)


def test_quantize_error_bound():
    x = synthetic.normal((100000,), tag=24) * 3
    s = ops.absmax_scale(np.abs(x).max())
    dq = ops.dequantize_int8(ops.quantize_int8(x, s), s)
    assert np.abs(x - dq).max() <= s / 2 * (1 + 1e-6)


def test_int8_accumulators_exact():
    rng = np.random.default_rng(0)
    a = rng.integers(-128, 128, (37, 3072)).astype(np.int8)
    w = rng.integers(-128, 128, (29, 3072)).astype(np.int8)
    a[0] = -128
    w[0] = -128
    np.testing.assert_array_equal(ops.int8_matmul_acc(a, w), ops.int8_matmul_acc_i64(a, w))
    assert ops.int8_matmul_acc(a, w)[0, 0] == 128 * 128 * 3072


def test_per_channel_weights_and_minmax():
    w = synthetic.normal((64, 768), tag=25, std=0.02)
    q, s = ops.quantize_weight_per_channel(w)
    np.testing.assert_allclose(s, np.abs(w).max(1) / 127, rtol=1e-7)
    assert (np.abs(q).max(1) == 127).all()
    obs = ops.MinMaxObserver()
    obs.update(np.array([-3.0, 1.0]))
    obs.update(np.array([2.0, 2.5]))
    assert obs.scale() == np.float32(3.0) / np.float32(127)
    assert ops.absmax_scale(0.0) == 1.0


# ------------------------------------------------------------ BERT layer ---
def _hf_layer(w, eps=1e-12):
    from transformers import BertConfig
    from transformers.models.bert.modeling_bert import BertLayer

    cfg = BertConfig(hidden_size=768, num_attention_heads=12, intermediate_size=3072,
                     hidden_act="gelu", layer_norm_eps=eps, hidden_dropout_prob=0.0,
                     attention_probs_dropout_prob=0.0)
    cfg._attn_implementation = "eager"
    layer = BertLayer(cfg).eval()
    sd = {
        "attention.self.query.weight": w["Wq"], "attention.self.query.bias": w["bq"],
        "attention.self.key.weight": w["Wk"], "attention.self.key.bias": w["bk"],
        "attention.self.value.weight": w["Wv"], "attention.self.value.bias": w["bv"],
        "attention.output.dense.weight": w["Wo"], "attention.output.dense.bias": w["bo"],
        "attention.output.LayerNorm.weight": w["ln1_g"], "attention.output.LayerNorm.bias": w["ln1_b"],
        "intermediate.dense.weight": w["Wi"], "intermediate.dense.bias": w["bi"],
        "output.dense.weight": w["Wo2"], "output.dense.bias": w["bo2"],
        "output.LayerNorm.weight": w["ln2_g"], "output.LayerNorm.bias": w["ln2_b"],
    }
    layer.load_state_dict({k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in sd.items()})
    return layer


def test_bert_layer_vs_transformers():
    w = synthetic.bert_weights(1, seed=3)[0]
    # non-trivial biases / LN params so every term is exercised
    for i, k in enumerate(("bq", "bk", "bv", "bo", "bi", "bo2", "ln1_b", "ln2_b")):
        w[k] = synthetic.normal(w[k].shape, tag=30 + i, std=0.1)
    w["ln1_g"] = synthetic.normal((768,), tag=40, std=0.1) + 1
    x = synthetic.hidden_states(2, 24, seed=3)
    lens = np.array([24, 9])
    layer = _hf_layer(w)
    mask = torch.zeros(2, 1, 1, 24)
    mask[1, ..., 9:] = torch.finfo(torch.float32).min
    with torch.no_grad():
        out = layer(torch.from_numpy(x), attention_mask=mask)
    hf = (out[0] if isinstance(out, tuple) else out).numpy()
    np.testing.assert_allclose(obert.bert_layer(x, w, lens), hf, rtol=1e-4, atol=2e-4)


def test_config1_golden():
    """Config 1 (one layer, b1 s128, fp32, seed 42): oracle vs the committed
    golden output produced by transformers.BertLayer (tests/golden/make_golden.py)."""
    g = np.load(os.path.join(GOLDEN, "config1_bert_layer.npz"))
    w = synthetic.bert_weights(1, seed=42)[0]
    x = synthetic.hidden_states(1, 128, seed=42)
    np.testing.assert_array_equal(x[0, :4, :4], g["x_corner"])  # seeded inputs unchanged
    np.testing.assert_allclose(obert.bert_layer(x, w), g["y"], rtol=1e-4, atol=2e-4)

"""The composed encoder's parity tests can fail: under the per-layer
LayerNorm / non-zero-bias weight set (synthetic.bert_weights_wired) every
wiring mistake the encoder's folded path could make moves the oracle's own
12-layer output by more than the 2e-2 bar those tests apply plus the
measured GPU-vs-oracle distance (about 1.1e-3 for the fp16 chain).

The mistakes are planted in the oracle's weights, on the CPU. Each stands
for one mistake in zenith_amd/encoder.py's host-side wiring:
  - a LayerNorm's gamma/beta taken from the neighbouring layer (the folded
    QKV projection applies the previous layer's LN2; FFN-up/down apply LN1),
  - the folded constant c = beta . W^T + b dropped (beta and the bias gone),
  - the per-head Q/K/V bias interleave wrong (query and key biases swapped,
    or every bias shifted by one head),
  - an epilogue bias dropped (out-projection or FFN-down).
Under the default weights (gamma 1, beta 0, biases 0 in every layer) each of
these leaves the output unchanged, which is checked too."""

import numpy as np
import pytest

from oracle import bert as obert
from zenith_amd import synthetic

BAR = 2e-2 + 5e-3  # the tests' bar plus margin for the GPU's own distance
B, S, NL = 2, 128, 12


def _r16(layers):
    return [{k: synthetic.round_f16(v) for k, v in w.items()} for w in layers]


def _shift_layer(layers, keys):
    out = [dict(w) for w in layers]
    for i in range(len(layers) - 1):
        for k in keys:
            out[i][k] = layers[i + 1][k]
    return out


def _zero(layers, keys):
    return [{k: (np.zeros_like(v) if k in keys else v) for k, v in w.items()} for w in layers]


def _swap_qk_bias(layers):
    return [dict(w, bq=w["bk"], bk=w["bq"]) for w in layers]


def _roll_head_bias(layers, D=64):
    return [dict(w, **{k: np.roll(w[k], D) for k in ("bq", "bk", "bv")}) for w in layers]


MISTAKES = {
    "ln2_from_next_layer": lambda w: _shift_layer(w, ("ln2_g", "ln2_b")),
    "ln2_gamma_from_next_layer": lambda w: _shift_layer(w, ("ln2_g",)),
    "ln1_from_next_layer": lambda w: _shift_layer(w, ("ln1_g", "ln1_b")),
    "qkv_fold_constant_dropped": lambda w: _zero(w, ("ln2_b", "bq", "bk", "bv")),
    "ffn_up_fold_constant_dropped": lambda w: _zero(w, ("ln1_b", "bi")),
    "qk_bias_swapped": _swap_qk_bias,
    "bias_shifted_one_head": _roll_head_bias,
    "out_proj_bias_dropped": lambda w: _zero(w, ("bo",)),
    "ffn_down_bias_dropped": lambda w: _zero(w, ("bo2",)),
}


@pytest.fixture(scope="module")
def inputs():
    x = synthetic.round_f16(synthetic.hidden_states(B, S, seed=42))
    lens = np.array([S, 70], np.int32)
    return x, lens


def _rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.fixture(scope="module")
def wired(inputs):
    x, lens = inputs
    w = _r16(synthetic.bert_weights_wired(NL))
    return w, obert.bert_encoder(x, w, lens)


@pytest.mark.parametrize("name", sorted(MISTAKES))
def test_wired_weights_expose_mistake(inputs, wired, name):
    x, lens = inputs
    w, ref = wired
    planted = obert.bert_encoder(x, MISTAKES[name](w), lens)
    assert _rel(planted, ref) > BAR, _rel(planted, ref)


@pytest.mark.parametrize("name", ["ln2_from_next_layer", "ln1_from_next_layer",
                                  "qkv_fold_constant_dropped", "qk_bias_swapped",
                                  "out_proj_bias_dropped"])
def test_default_weights_hide_mistake(inputs, name):
    """Why the wired set exists: gamma 1 / beta 0 / zero biases in every layer
    make these mistakes invisible."""
    x, lens = inputs
    w = _r16(synthetic.bert_weights(NL))
    ref = obert.bert_encoder(x, w, lens)
    assert _rel(obert.bert_encoder(x, MISTAKES[name](w), lens), ref) == 0.0


def test_wired_weights_distributions():
    w = synthetic.bert_weights_wired(NL)
    base = synthetic.bert_weights(NL)
    for a, b in zip(w, base):
        for k in ("Wq", "Wk", "Wv", "Wo", "Wi", "Wo2"):
            np.testing.assert_array_equal(a[k], b[k])
        assert 0.08 < np.std(a["ln1_g"]) < 0.12 and abs(np.mean(a["ln2_g"]) - 1) < 0.02
        assert 0.4 < np.std(a["bq"]) < 0.6 and 0.04 < np.std(a["bi"]) < 0.06
    assert not np.array_equal(w[0]["ln2_g"], w[1]["ln2_g"])

"""GPU parity: BERT encoder (configs 1 and 5) through the fused HIP path vs
the oracle's fp32 encoder on the same fp16-rounded weights and inputs.
Bar: norm-relative error <= 2e-2 and |y - ref| <= 2e-2 + 2e-2 |ref|."""

import functools

import numpy as np
import pytest
import torch

from oracle import bert as obert
from oracle import ops
from tests.conftest import fp16_tol
from zenith_amd import synthetic

pytestmark = pytest.mark.gpu


def _check(y, ref, bar=2e-2, elementwise=True):
    rel = float(np.linalg.norm(y - ref) / np.linalg.norm(ref))
    worst = float(np.max(np.abs(y - ref) - (bar + bar * np.abs(ref)))) if elementwise else -1.0
    assert rel <= bar and worst <= 0, (rel, worst)
    return rel


def _r16(layers):
    return [{k: synthetic.round_f16(v) for k, v in w.items()} for w in layers]


# "default": the workload configs' weights (gamma 1, beta 0, biases 0 in every
# layer). "wired": per-layer LayerNorm parameters and non-zero biases
# (synthetic.bert_weights_wired), under which taking a LayerNorm from the
# wrong layer, dropping a folded beta/bias constant or mis-interleaving the
# per-head Q/K/V bias moves the output past the bar (tests/test_wiring_weights.py
# plants each such mistake in the oracle).
WEIGHTS = {"default": synthetic.bert_weights, "wired": synthetic.bert_weights_wired}


@functools.lru_cache(maxsize=4)
def _weights(kind, n=12):
    return _r16(WEIGHTS[kind](n, seed=42))


@pytest.mark.parametrize("kind", sorted(WEIGHTS))
def test_config1_single_layer(dev, kind):
    from zenith_amd.encoder import BertEncoder

    w = _weights(kind, 1)
    x = synthetic.round_f16(synthetic.hidden_states(1, 128, seed=42))
    enc = BertEncoder(w, device=dev)
    y = enc(torch.from_numpy(x).to(dev, torch.float16)).float().cpu().numpy()
    _check(y, obert.bert_encoder(x, w))


FP16_CASES = ([("default",) + c for c in [(128, True, True), (128, False, True), (128, True, False),
                                          (512, False, True), (512, False, False)]]
              + [("wired",) + c for c in [(128, True, True), (128, False, True), (128, True, False),
                                          (128, False, False), (512, False, True),
                                          (512, False, False)]])


@pytest.mark.parametrize("kind,S,fused,fold", FP16_CASES)
def test_config5_encoder_fp16(dev, kind, S, fused, fold):
    """12 layers, B=32, lengths ~ U{S/2..S}, against the fp32 oracle: every
    sequence at S=128, with the fused QKV + attention launch (the default at
    S=128) and with the separate GEMM and attention kernels, with the
    LayerNorms folded into the GEMMs (the default) and as separate kernels;
    at S=512 eight sequences spread over the batch (the full batch is covered
    bit-exactly by the permutation test below). Both weight sets."""
    from zenith_amd.encoder import BertEncoder

    B = 32
    w = _weights(kind)
    x = synthetic.round_f16(synthetic.hidden_states(B, S, seed=42))
    lens = synthetic.padding_lengths(B, S)
    enc = BertEncoder(w, device=dev, fuse_qkv_attention=fused, fold_layernorm=fold)
    assert enc.fused_attention(S) == fused and enc.fold_ln == fold
    y = enc(torch.from_numpy(x).to(dev, torch.float16), torch.from_numpy(lens).to(dev)).float().cpu().numpy()
    assert np.isfinite(y).all()
    pick = np.arange(B) if S == 128 else np.array([0, 5, 9, 14, 18, 23, 27, 31])
    rel = _check(y[pick], obert.bert_encoder(x[pick], w, lens[pick]))
    two = pick[[0, -1]]
    rel16 = _check(y[two], obert.bert_encoder(x[two], w, lens[two], act_f16=True))
    print(f"encoder {kind} S={S} fused={fused} fold={fold}: rel vs fp32 oracle {rel:.3e} "
          f"({len(pick)} sequences), vs fp16-storage oracle {rel16:.3e}")


@pytest.mark.parametrize("B", [1, 4])
def test_small_batch_encoder(dev, B):
    """One and four sequences of 128 tokens (the reference's own BERT
    benchmark shape, and one rank's share of a batch of 32 over eight GPUs):
    the small-batch path (unfolded layers, 64x64 GEMM tiles with split-K
    through a workspace, one-wavefront attention workgroups) on the wired
    weights, every sequence against the fp32 oracle at the encoder bar; a
    HIP-graph replay gives the eager output bit for bit."""
    from zenith_amd.encoder import BertEncoder

    S = 128
    w = _weights("wired")
    x = synthetic.round_f16(synthetic.hidden_states(B, S, seed=5))
    lens = synthetic.padding_lengths(B, S, seed=5)
    enc = BertEncoder(w, device=dev)
    assert enc.small_batch(B, S) and not enc.folded(S, B) and not enc.fused_attention(S, B)
    xt = torch.from_numpy(x).to(dev, torch.float16)
    lt = torch.from_numpy(lens).to(dev)
    y = enc(xt, lt)
    assert enc._bufs["ws"] is not None  # some product is split at this size
    yn = y.float().cpu().numpy()
    rel = _check(yn, obert.bert_encoder(x, w, lens))
    gx, gl, go = enc.capture(B, S)
    gx.copy_(xt)
    gl.copy_(lt)
    enc.replay()
    torch.cuda.synchronize()
    assert torch.equal(go, y)
    print(f"small-batch encoder b{B} s{S}: rel vs fp32 oracle {rel:.3e}")


@pytest.mark.parametrize("S,int8", [(128, False), (512, False), (128, True), (512, True)])
def test_config5_batch_permutation_invariance(dev, S, int8):
    """The B=32 batch run in reversed order gives every sequence's output
    bit-identical to the forward order: each output row depends only on its
    own sequence, through kernels whose K-reduction order does not depend on
    where a row or a (batch, head) lands in the grid. A batch-indexing error
    (a wrong length, head or row offset for some batch entries) breaks it."""
    from zenith_amd.encoder import BertEncoder

    B = 32
    w = _weights("wired")
    x = synthetic.round_f16(synthetic.hidden_states(B, S, seed=42))
    lens = synthetic.padding_lengths(B, S)
    enc = BertEncoder(w, device=dev)
    if int8:
        enc.enable_int8_ffn([4.5 / 127] * 12, [6.0 / 127] * 12, layers_fp32=w)
    perm = np.arange(B)[::-1].copy()
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    y = enc(T(x).half(), T(lens))
    yp = enc(T(x[perm]).half(), T(lens[perm]))
    assert torch.equal(yp, y[torch.from_numpy(perm).to(dev)])


# Eight sequences spread over the batch for the INT8 chain checks.
INT8_PICK = np.array([0, 3, 9, 14, 18, 23, 27, 31])
INT8_CASES = [("default", 128, True), ("default", 512, False), ("default", 128, False),
              ("wired", 128, True), ("wired", 512, False)]


@functools.lru_cache(maxsize=4)
def _int8_setup(kind, S):
    """Weights, inputs, the fp32 oracle's output on the picked sequences, and
    per-layer activation scales calibrated on the fp32 oracle's activations
    of those sequences (absmax/127 of the FFN input and of the GELU output),
    with the oracle's int8 operands for every layer."""
    B = 32
    w = _weights(kind)
    x = synthetic.round_f16(synthetic.hidden_states(B, S, seed=42))
    lens = synthetic.padding_lengths(B, S)
    s_x, s_h = [], []
    h = x[INT8_PICK]
    for lw in w:
        taps = {}
        h = obert.bert_layer(h, lw, lens[INT8_PICK], taps=taps)
        s_x.append(float(ops.absmax_scale(np.abs(taps["h1"]).max())))
        s_h.append(float(ops.absmax_scale(np.abs(taps["u"]).max())))
    int8_layers = []
    for i, lw in enumerate(w):
        qi, si = ops.quantize_weight_per_channel(lw["Wi"])
        qo, so = ops.quantize_weight_per_channel(lw["Wo2"])
        int8_layers.append({"Wi_q": qi, "s_wi": si, "Wo2_q": qo, "s_wo2": so,
                            "s_x": np.float32(s_x[i]), "s_h": np.float32(s_h[i])})
    return w, x, lens, s_x, s_h, int8_layers, h


def _int8_encoder(dev, w, s_x, s_h, fold):
    from zenith_amd.encoder import BertEncoder

    enc = BertEncoder(w, device=dev, fold_layernorm=fold)
    enc.enable_int8_ffn(s_x, s_h, layers_fp32=w)
    return enc


def _f16(a):
    return a.astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("kind,S,fold", INT8_CASES)
def test_config5_int8_ffn_per_layer(dev, kind, S, fold):
    """INT8-FFN variant at B=32, S=128 and S=512, on eight sequences, layer
    by layer along the GPU's own trajectory (every GPU layer's input is the
    previous GPU layer's output), and inside each layer stage by stage from
    the GPU's own intermediate tensors, so that each stage is checked on
    exactly the operands it consumed:
      1. LN1's output h1 against the oracle layer's (same input, fp16
         storage) at the fp16 bar;
      2. its int8 copy bit-exact against quantising the GPU's h1;
      3. the re-quantised GELU output against the oracle's dequant + bias +
         GELU + quantise of the GPU's int8 input (the int32 accumulators are
         exact): every difference is one step, at an element whose fp16 GELU
         value lies within one fp16 ulp of an int8 rounding boundary;
      4. the FFN-down output against the oracle's on the GPU's int8 GELU
         output at the fp16 bar (with the residual h1 where the layer is
         folded);
      5. the layer output against the oracle's LN2 of the GPU's FFN-down
         output at the fp16 bar;
    and the whole layer against the oracle layer on the same input at the
    north-star 2e-2 norm-relative bar. Whole-layer elementwise comparison is
    not a bar here: a one-ulp difference in h1 (the attention's fp16
    products) that crosses an int8 rounding boundary shifts ~80 GELU outputs
    of that row by one step, and the row of the FFN-down output by up to
    ~2e-2, which stage 2-4 account for exactly. With the LayerNorms folded
    (the default at S=128) and unfolded (as the INT8-FFN encoder runs at
    S=512)."""
    w, x, lens, s_x, s_h, int8_layers, _ = _int8_setup(kind, S)
    enc = _int8_encoder(dev, w, s_x, s_h, fold)
    assert enc.folded(S) == fold
    for i in range(len(w)):
        # the encoder's torch-side weight quantiser agrees with the oracle's
        np.testing.assert_array_equal(enc.int8[i]["Wi_q"].cpu().numpy(), int8_layers[i]["Wi_q"])
        np.testing.assert_array_equal(enc.int8[i]["Wo2_q"].cpu().numpy(), int8_layers[i]["Wo2_q"])
    h = x[INT8_PICK]
    lp = torch.from_numpy(lens[INT8_PICK]).to(dev)
    worst, flips, n_u = 0.0, 0, 0
    for i, lw in enumerate(w):
        il = int8_layers[i]
        taps = {}
        ref_i = obert.bert_layer(h, lw, lens[INT8_PICK], int8=il, act_f16=True, taps=taps)
        y_i = enc.forward_layers(torch.from_numpy(h).to(dev, torch.float16), lp, i, i + 1)
        y_i = y_i.float().cpu().numpy()
        tn = enc.int8_ffn_tensors(i)
        M = y_i.shape[0] * y_i.shape[1]
        g_h1 = tn["h1"][:M].float().cpu().numpy()
        g_qh = tn["q_h"][:M].cpu().numpy()
        g_qu = tn["q_u"][:M].cpu().numpy()
        g_out = tn["ffn_out"][:M].float().cpu().numpy()
        # 1. attention half
        ok, ex = fp16_tol(g_h1, taps["h1"])
        assert ok, ("h1", i, ex)
        # 2. FFN input quantisation, bit-exact
        np.testing.assert_array_equal(g_qh, ops.quantize_int8(g_h1, il["s_x"]))
        # 3. FFN-up + GELU + requantisation on the GPU's own int8 input
        u = _f16(ops.int8_linear(g_qh, il["Wi_q"], il["s_x"], il["s_wi"], lw["bi"], "gelu"))
        qu = ops.quantize_int8(u, il["s_h"])
        diff = g_qu.astype(np.int32) - qu
        assert np.abs(diff).max(initial=0) <= 1, ("q_u step", i)
        bad = diff != 0
        if bad.any():
            t = u[bad] / np.float32(il["s_h"])
            to_boundary = np.abs(np.abs(t - np.rint(t)) - 0.5)
            ulp = np.spacing(np.abs(u[bad]).astype(np.float16)).astype(np.float32) / np.float32(il["s_h"])
            assert np.all(to_boundary <= 1.01 * ulp), ("q_u flip away from a boundary", i)
        flips += int(bad.sum())
        n_u += bad.size
        # 4. FFN-down on the GPU's own int8 GELU output
        d = ops.int8_linear(g_qu, il["Wo2_q"], il["s_h"], il["s_wo2"], lw["bo2"])
        d = _f16(d + g_h1) if tn["residual"] else _f16(d)
        ok, ex = fp16_tol(g_out, d)
        assert ok, ("ffn_out", i, ex)
        # 5. LN2 of the GPU's FFN-down output
        ln2 = (ops.layernorm(g_out, lw["ln2_g"], lw["ln2_b"], 1e-12) if tn["residual"]
               else ops.add_layernorm(g_out, g_h1, lw["ln2_g"], lw["ln2_b"], 1e-12))
        ok, ex = fp16_tol(y_i.reshape(M, -1), ln2)
        assert ok, ("layer output", i, ex)
        # the whole layer
        worst = max(worst, _check(y_i, ref_i, elementwise=False))
        h = y_i
    print(f"int8 {kind} S={S} fold={fold}: worst per-layer rel {worst:.3e}; "
          f"GELU requantisation flips {flips} of {n_u} ({flips / n_u:.2e}), all at boundaries")


@pytest.mark.parametrize("kind,S,fold", INT8_CASES)
def test_config5_int8_ffn_end_to_end(dev, kind, S, fold):
    """The 12-layer INT8 chain end to end on eight sequences. The chain is
    ill-conditioned at the last-bit level: an activation whose fp16 value
    differs in the last bit can fall on the other side of an int8 rounding
    boundary (a whole quantisation step for that element), and later layers
    amplify that. The oracle itself, given its own input perturbed by half an
    fp16 ulp, moves by ~3e-2 over 12 layers (its fp16 chain by ~1e-3). The
    GPU chain is therefore held to the oracle's measured self-sensitivity
    (median over three perturbation seeds, with 25% margin) or 2e-2,
    whichever is larger; the ratio of the two is printed. Against the fp32
    (not quantised) model the chain stays within 0.1."""
    w, x, lens, s_x, s_h, int8_layers, ref32 = _int8_setup(kind, S)
    enc = _int8_encoder(dev, w, s_x, s_h, fold)
    y = enc(torch.from_numpy(x).to(dev, torch.float16), torch.from_numpy(lens).to(dev)).float().cpu().numpy()
    y = y[INT8_PICK]
    xp, lp = x[INT8_PICK], lens[INT8_PICK]
    ref = obert.bert_encoder(xp, w, lp, int8_layers=int8_layers, act_f16=True)
    rel = float(np.linalg.norm(y - ref) / np.linalg.norm(ref))
    worst = float(np.max(np.abs(y - ref) - (2e-2 + 2e-2 * np.abs(ref))))
    sens = []
    for seed in (0, 1, 2):
        noise = np.random.default_rng(seed).standard_normal(xp.shape).astype(np.float32)
        ref_p = obert.bert_encoder(xp * (1 + noise * np.float32(2.0 ** -11)), w, lp,
                                   int8_layers=int8_layers, act_f16=True)
        sens.append(float(np.linalg.norm(ref_p - ref) / np.linalg.norm(ref)))
    self_sens = float(np.median(sens))
    rel32 = float(np.linalg.norm(y - ref32) / np.linalg.norm(ref32))
    print(f"int8 encoder {kind} S={S} fold={fold}: rel vs int8 oracle {rel:.3e} "
          f"(elementwise excess {worst:.3e}); oracle self-sensitivity "
          f"{', '.join(f'{s:.3e}' for s in sens)} (median {self_sens:.3e}); "
          f"ratio {rel / self_sens:.3f}; vs fp32 model {rel32:.3e}")
    assert rel <= max(2e-2, 1.25 * self_sens), (rel, sens, worst)
    assert rel32 < 0.1


def test_graph_replay_matches_eager(dev):
    """HIP-graph replays (several, with eager work in between) reproduce the
    eager forward bit-for-bit."""
    from zenith_amd.encoder import BertEncoder

    B, S = 8, 128
    w = _r16(synthetic.bert_weights(2, seed=7))
    x = torch.from_numpy(synthetic.round_f16(synthetic.hidden_states(B, S, seed=7))).to(dev, torch.float16)
    lens = torch.from_numpy(synthetic.padding_lengths(B, S, seed=7)).to(dev)
    enc = BertEncoder(w, device=dev)
    eager = enc(x, lens).clone()
    gx, gl, go = enc.capture(B, S)
    for i in range(3):
        gx.copy_(x)
        gl.copy_(lens)
        enc.replay()
        torch.cuda.synchronize()
        assert torch.equal(go, eager), f"replay {i} differs"
        _ = enc(x * 0.5, lens)  # eager work between replays
        torch.cuda.synchronize()

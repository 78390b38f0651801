"""GPU parity: the FFN intermediate in fragment order.

- zk_gemm_f16_res_stats_frag reads A in fragment order (each lane loads its
  MFMA A fragments straight from memory) and must give zk_gemm_f16_res_stats's
  output and statistics bit for bit, on the same rows in row-major order,
  wherever both run the 128x96 tile; the padding rows of the
  fragment-ordered A (past M) are filled with NaN, which must reach no stored
  value. Where zk_gemm_f16_res_stats takes its 256x192 tile (M = 16384,
  N = 768) the two launches' results are not bit-identical (the frag entry
  always runs the 128x96 tile), and the frag result is checked against the
  oracle at the fp16 bar instead, as is one other shape.
- zk_gemm_f16_ln_frag writes zk_gemm_f16_ln's GELU output (bit for bit) in
  fragment order, on every tile configuration it runs (256x256, 256x192,
  128x128 and the 128x96 tile that replaces the 16x16-MFMA ones), and leaves
  the padding rows past M untouched.
- The int8 pair: zk_gemm_i8_requant_frag writes zk_gemm_i8_requant's int8
  values in fragment order (32 columns per k-step), bit for bit, rows past M
  untouched; zk_gemm_i8_res_stats_frag gives zk_gemm_i8_res_stats's output
  and statistics bit for bit on the same tile.
- zk_qkv_attn_f16_frag writes zk_qkv_attn_f16's / zk_qkv_attn_f16_ln's
  attention output, bit for bit, in fragment order (padding rows untouched).
- The folded encoder with and without the fragment-ordered FFN and attention
  output gives the same output, bit for bit, in fp16 and with the INT8 FFN.
"""

import math

import numpy as np
import pytest
import torch

from oracle import ops
from tests.conftest import fp16_tol
from zenith_amd import _lib as L
from zenith_amd import synthetic
from zenith_amd.encoder import (BertEncoder, fold_layernorm, from_fragment_order,
                                to_fragment_order)

pytestmark = pytest.mark.gpu

SEG = 96
EPS = 1e-12


def _t(a, dev, dtype=torch.float16):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev, dtype)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _res_stats(name, a_ptr, lda, tw, tb, tr, st, tg, tbe, M, N, K, dev):
    c = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    part = torch.full((M, N // SEG, 2), float("nan"), dtype=torch.float32, device=dev)
    ln = st is not None
    head = (a_ptr, tw.data_ptr(), c.data_ptr(), M, N, K) + ((lda,) if lda else ()) + (K, N)
    L.call(name, *head, tb.data_ptr(), tr.data_ptr(), N, st.data_ptr() if ln else None,
           tg.data_ptr() if ln else None, tbe.data_ptr() if ln else None, part.data_ptr(),
           _stream())
    torch.cuda.synchronize()
    return c, part


@pytest.mark.parametrize("M,K,N", [(4096, 3072, 768), (1000, 3072, 768), (4096, 768, 768),
                                   (100, 64, 96), (300, 256, 288), (16384, 3072, 768)])
@pytest.mark.parametrize("ln_res", [False, True])
def test_res_stats_frag_matches_row_major(dev, M, K, N, ln_res):
    a = synthetic.round_f16(synthetic.normal((M, K), tag=180))
    w = synthetic.round_f16(synthetic.normal((N, K), tag=181, std=1.0 / math.sqrt(K)))
    b = synthetic.round_f16(synthetic.normal((N,), tag=182, std=0.1))
    res = synthetic.round_f16(synthetic.normal((M, N), tag=183))
    g = synthetic.round_f16(1.0 + synthetic.normal((N,), tag=184, std=0.2))
    be = synthetic.round_f16(synthetic.normal((N,), tag=185, std=0.2))
    ta, tw, tb, tr, tg, tbe = (_t(v, dev) for v in (a, w, b, res, g, be))
    st = None
    if ln_res:
        r64 = res.astype(np.float64)
        st = _t(np.stack([r64.mean(1), 1.0 / np.sqrt(r64.var(1) + EPS)], -1), dev,
                torch.float32)
    af = to_fragment_order(ta)
    Mp = -(-M // 32) * 32
    if Mp > M:  # padding rows: read, never stored
        af.view(Mp // 32, K // 16, 2, 32, 8)[-1, :, :, M % 32:, :] = float("nan")
    print(f"zk_gemm_f16_res_stats_frag M={M} K={K} N={N} ln_res={ln_res}", flush=True)
    c0, p0 = _res_stats("zk_gemm_f16_res_stats", ta.data_ptr(), K, tw, tb, tr, st, tg, tbe,
                        M, N, K, dev)
    c1, p1 = _res_stats("zk_gemm_f16_res_stats_frag", af.data_ptr(), 0, tw, tb, tr, st, tg,
                        tbe, M, N, K, dev)
    assert not torch.isnan(c1).any()
    same_tile = not (M >= 1024 and N % 192 == 0 and -(-M // 256) * (N // 192) >= 160)
    if same_tile:
        assert torch.equal(c0.view(torch.int16), c1.view(torch.int16))
        assert torch.equal(p0.view(torch.int32), p1.view(torch.int32))
    if (M, K, N) == (1000, 3072, 768) or not same_tile:
        r = res
        if ln_res:
            s = st.cpu().numpy()
            r = (res - s[:, :1]) * s[:, 1:] * g + be
        ok, worst = fp16_tol(c1.float().cpu().numpy(), ops.linear(a, w, b) + r)
        assert ok, worst


def _ln_frag_case(dev, M, K, N):
    x = synthetic.round_f16(synthetic.normal((M, K), tag=190) * 1.5 + 0.3)
    w = synthetic.round_f16(synthetic.normal((N, K), tag=191, std=1.0 / math.sqrt(K)))
    b = synthetic.round_f16(synthetic.normal((N,), tag=192, std=0.1))
    g = synthetic.round_f16(1.0 + synthetic.normal((K,), tag=193, std=0.2))
    be = synthetic.round_f16(synthetic.normal((K,), tag=194, std=0.2))
    wf, s, cc = fold_layernorm(w, b, g, be)
    x64 = x.astype(np.float64).reshape(M, K // SEG, SEG)
    mean = x64.mean(-1)
    part = np.stack([mean, ((x64 - mean[..., None]) ** 2).sum(-1)], -1).astype(np.float32)
    tx, twf = _t(x, dev), _t(wf, dev)
    tp, ts, tc = (_t(v, dev, torch.float32) for v in (part, s, cc))
    return tx, twf, tp, ts, tc


@pytest.mark.parametrize("M,K,N", [(4096, 768, 3072), (16384, 768, 3072), (1000, 96, 10240),
                                   (2048, 768, 3072), (100, 96, 128), (300, 288, 192)])
def test_ln_frag_matches_row_major(dev, M, K, N):
    tx, twf, tp, ts, tc = _ln_frag_case(dev, M, K, N)
    out = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    mr0 = torch.full((M, 2), float("nan"), dtype=torch.float32, device=dev)
    mr1 = torch.full((M, 2), float("nan"), dtype=torch.float32, device=dev)
    Mp = -(-M // 32) * 32
    fr = torch.full((Mp * N,), 7.0, dtype=torch.float16, device=dev)
    print(f"zk_gemm_f16_ln_frag M={M} K={K} N={N}", flush=True)
    L.call("zk_gemm_f16_ln", tx.data_ptr(), twf.data_ptr(), out.data_ptr(), M, N, K, K, K, N,
           tp.data_ptr(), EPS, ts.data_ptr(), tc.data_ptr(), mr0.data_ptr(),
           L.ZK_EPI_BIAS_GELU_ERF, _stream())
    L.call("zk_gemm_f16_ln_frag", tx.data_ptr(), twf.data_ptr(), fr.data_ptr(), M, N, K, K, K,
           tp.data_ptr(), EPS, ts.data_ptr(), tc.data_ptr(), mr1.data_ptr(), _stream())
    torch.cuda.synchronize()
    y = from_fragment_order(fr, M, N)
    assert torch.equal(y.view(torch.int16), out.view(torch.int16))
    assert torch.equal(mr0.view(torch.int32), mr1.view(torch.int32))
    if Mp > M:  # rows past M are not written
        pad = fr.view(Mp // 32, N // 16, 2, 32, 8)[-1, :, :, M % 32:, :]
        assert bool((pad == 7.0).all())


def test_frag_shape_errors(dev):
    t = torch.zeros(1 << 16, dtype=torch.float16, device=dev)
    f = torch.zeros(1 << 12, dtype=torch.float32, device=dev)
    p = t.data_ptr()
    lib = L.load()
    # K not a multiple of 64 (fragment-ordered A is read in 64-deep slices)
    rc = lib.zk_gemm_f16_res_stats_frag(p, p, p, 32, 96, 96, 96, 96, p, p, 96, None, None, None,
                                        f.data_ptr(), _stream())
    assert rc == L.ZK_ERR_UNSUPPORTED, L.last_error()
    # N not a multiple of 64 (the consumer's K)
    rc = lib.zk_gemm_f16_ln_frag(p, p, p, 32, 96, 96, 96, 96, f.data_ptr(), EPS, f.data_ptr(),
                                 f.data_ptr(), None, _stream())
    assert rc == L.ZK_ERR_UNSUPPORTED, L.last_error()
    torch.cuda.synchronize()


@pytest.mark.parametrize("B,S", [(32, 128), (33, 64), (17, 128)])
def test_encoder_frag_ffn_bit_identical(dev, B, S):
    """B x S rows: whole 256-row tiles (b32 s128), and ragged last tiles
    (2112 and 2176 rows) whose fused-attention waves past the batch store
    nothing."""
    layers = synthetic.bert_weights_wired(3, seed=7)
    x = torch.from_numpy(synthetic.hidden_states(B, S, seed=7)).to(dev, torch.float16)
    lens = torch.from_numpy(synthetic.padding_lengths(B, S)).to(dev)
    outs = []
    print(f"encoder fragment order on/off B={B} S={S}", flush=True)
    for frag in (True, False):
        enc = BertEncoder(layers, device=dev)
        enc.ffn_frag = frag
        enc.attn_frag = frag
        assert enc.frag_ffn(B * S) == frag
        outs.append(enc.forward(x, lens).clone())
        torch.cuda.synchronize()
        if frag:
            assert enc._bufs["u_frag"] is not None and enc._bufs["ctx_frag"] is not None
        del enc
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


def _i8(shape, tag):
    return np.clip(np.rint(synthetic.normal(shape, tag=tag) * 40), -127, 127).astype(np.int8)


@pytest.mark.parametrize("M,K,N", [(4096, 768, 3072), (1000, 768, 3072), (100, 256, 384),
                                   (300, 128, 256)])
def test_i8_requant_frag_matches_row_major(dev, M, K, N):
    qa, qw = _t(_i8((M, K), 200), dev, torch.int8), _t(_i8((N, K), 201), dev, torch.int8)
    sw = _t(np.abs(synthetic.normal((N,), tag=202, std=1e-3)) + 5e-4, dev, torch.float32)
    b = _t(synthetic.round_f16(synthetic.normal((N,), tag=203, std=0.1)), dev)
    s_x, s_out = 0.02, 6.0 / 127
    q0 = torch.full((M, N), 99, dtype=torch.int8, device=dev)
    Mp = -(-M // 32) * 32
    q1 = torch.full((Mp * N,), 99, dtype=torch.int8, device=dev)
    print(f"zk_gemm_i8_requant_frag M={M} K={K} N={N}", flush=True)
    L.call("zk_gemm_i8_requant", qa.data_ptr(), qw.data_ptr(), q0.data_ptr(), M, N, K, K, K, N,
           s_x, sw.data_ptr(), b.data_ptr(), L.ZK_EPI_BIAS_GELU_ERF, s_out, _stream())
    L.call("zk_gemm_i8_requant_frag", qa.data_ptr(), qw.data_ptr(), q1.data_ptr(), M, N, K, K, K,
           s_x, sw.data_ptr(), b.data_ptr(), L.ZK_EPI_BIAS_GELU_ERF, s_out, _stream())
    torch.cuda.synchronize()
    assert torch.equal(from_fragment_order(q1, M, N), q0)
    if Mp > M:  # rows past M are not written
        pad = q1.view(Mp // 32, N // 32, 2, 32, 16)[-1, :, :, M % 32:, :]
        assert bool((pad == 99).all())


@pytest.mark.parametrize("M,K,N", [(4096, 3072, 768), (1000, 3072, 768), (300, 256, 288)])
@pytest.mark.parametrize("ln_res", [False, True])
def test_i8_res_stats_frag_matches_row_major(dev, M, K, N, ln_res):
    qa, qw = _t(_i8((M, K), 210), dev, torch.int8), _t(_i8((N, K), 211), dev, torch.int8)
    sw = _t(np.abs(synthetic.normal((N,), tag=212, std=1e-4)) + 5e-5, dev, torch.float32)
    b = _t(synthetic.round_f16(synthetic.normal((N,), tag=213, std=0.1)), dev)
    res = _t(synthetic.round_f16(synthetic.normal((M, N), tag=214)), dev)
    g = _t(synthetic.round_f16(1.0 + synthetic.normal((N,), tag=215, std=0.2)), dev)
    be = _t(synthetic.round_f16(synthetic.normal((N,), tag=216, std=0.2)), dev)
    r64 = res.double()
    st = torch.stack([r64.mean(1), 1.0 / torch.sqrt(r64.var(1, unbiased=False) + EPS)], 1).float()
    af = to_fragment_order(qa)
    Mp = -(-M // 32) * 32
    if Mp > M:  # padding rows: read, never stored
        af.view(Mp // 32, K // 32, 2, 32, 16)[-1, :, :, M % 32:, :] = 127
    outs = []
    print(f"zk_gemm_i8_res_stats_frag M={M} K={K} N={N} ln_res={ln_res}", flush=True)
    for frag in (False, True):
        c = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
        part = torch.full((M, N // SEG, 2), float("nan"), dtype=torch.float32, device=dev)
        ln = (st.data_ptr(), g.data_ptr(), be.data_ptr()) if ln_res else (None, None, None)
        if frag:
            L.call("zk_gemm_i8_res_stats_frag", af.data_ptr(), qw.data_ptr(), c.data_ptr(), M, N,
                   K, K, N, 0.01, sw.data_ptr(), b.data_ptr(), res.data_ptr(), N, *ln,
                   part.data_ptr(), _stream())
        else:
            L.call("zk_gemm_i8_res_stats", qa.data_ptr(), qw.data_ptr(), c.data_ptr(), M, N, K, K,
                   K, N, 0.01, sw.data_ptr(), b.data_ptr(), res.data_ptr(), N, *ln,
                   part.data_ptr(), _stream())
        torch.cuda.synchronize()
        outs.append((c, part))
    (c0, p0), (c1, p1) = outs
    assert not torch.isnan(c1).any()
    assert torch.equal(c0.view(torch.int16), c1.view(torch.int16))
    assert torch.equal(p0.view(torch.int32), p1.view(torch.int32))


def test_encoder_int8_frag_ffn_bit_identical(dev):
    layers = synthetic.bert_weights_wired(3, seed=9)
    B, S = 32, 128
    x = torch.from_numpy(synthetic.hidden_states(B, S, seed=9)).to(dev, torch.float16)
    lens = torch.from_numpy(synthetic.padding_lengths(B, S)).to(dev)
    outs = []
    for frag in (True, False):
        enc = BertEncoder(layers, device=dev)
        enc.ffn_frag = frag
        enc.enable_int8_ffn([0.05] * 3, [6.0 / 127] * 3, layers_fp32=layers)
        outs.append(enc.forward(x, lens).clone())
        torch.cuda.synchronize()
        assert (enc._bufs["q_u_frag"] is not None) == frag
        del enc
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


@pytest.mark.parametrize("B,S", [(32, 128), (5, 128), (3, 64)])
@pytest.mark.parametrize("ln", [False, True])
def test_qkv_attn_frag_matches_row_major(dev, B, S, ln):
    heads, H = 12, 768
    M = B * S
    x = _t(synthetic.round_f16(synthetic.normal((M, H), tag=220)), dev)
    w = _t(synthetic.round_f16(synthetic.normal((3 * H, H), tag=221, std=0.05)), dev)
    b = _t(synthetic.round_f16(synthetic.normal((3 * H,), tag=222, std=0.1)), dev)
    lens = torch.from_numpy(synthetic.padding_lengths(B, S)).to(dev)
    xn = x.double().cpu().numpy().reshape(M, H // SEG, SEG)
    mean = xn.mean(-1)
    part = _t(np.stack([mean, ((xn - mean[..., None]) ** 2).sum(-1)], -1), dev, torch.float32)
    sc = _t(synthetic.normal((3 * H,), tag=223, std=0.1), dev, torch.float32)
    cc = _t(synthetic.normal((3 * H,), tag=224, std=0.1), dev, torch.float32)
    Mp = -(-M // 32) * 32
    c0 = torch.full((M, H), float("nan"), dtype=torch.float16, device=dev)
    c1 = torch.full((Mp * H,), 7.0, dtype=torch.float16, device=dev)
    scale = 1.0 / math.sqrt(64)
    print(f"zk_qkv_attn_f16_frag B={B} S={S} ln={ln}", flush=True)
    if ln:
        L.call("zk_qkv_attn_f16_ln", x.data_ptr(), w.data_ptr(), part.data_ptr(), EPS,
               sc.data_ptr(), cc.data_ptr(), None, c0.data_ptr(), B, S, H, heads, lens.data_ptr(),
               scale, _stream())
    else:
        L.call("zk_qkv_attn_f16", x.data_ptr(), w.data_ptr(), b.data_ptr(), c0.data_ptr(), B, S,
               H, heads, lens.data_ptr(), scale, _stream())
    L.call("zk_qkv_attn_f16_frag", x.data_ptr(), w.data_ptr(), b.data_ptr(),
           part.data_ptr() if ln else None, EPS, sc.data_ptr() if ln else None,
           cc.data_ptr() if ln else None, None, c1.data_ptr(), B, S, H, heads, lens.data_ptr(),
           scale, _stream())
    torch.cuda.synchronize()
    assert torch.equal(from_fragment_order(c1, M, H).view(torch.int16), c0.view(torch.int16))
    if Mp > M:
        pad = c1.view(Mp // 32, H // 16, 2, 32, 8)[-1, :, :, M % 32:, :]
        assert bool((pad == 7.0).all())


@pytest.mark.parametrize("M,K,N", [(4096, 3072, 768), (1000, 3072, 768), (4096, 768, 768)])
def test_gemm_f16_frag(dev, M, K, N):
    """zk_gemm_f16_frag (A in fragment order, bias, the 128x96 tile): bit for
    bit with zk_gemm_f16 where that runs the same tile (K >= 2048 at
    N <= 1024), and at the fp16 bar against the oracle at the out-projection
    shape, where zk_gemm_f16 takes 64x64 tiles."""
    a = synthetic.round_f16(synthetic.normal((M, K), tag=230))
    w = synthetic.round_f16(synthetic.normal((N, K), tag=231, std=1.0 / math.sqrt(K)))
    b = synthetic.round_f16(synthetic.normal((N,), tag=232, std=0.1))
    ta, tw, tb = _t(a, dev), _t(w, dev), _t(b, dev)
    af = to_fragment_order(ta)
    Mp = -(-M // 32) * 32
    if Mp > M:
        af.view(Mp // 32, K // 16, 2, 32, 8)[-1, :, :, M % 32:, :] = float("nan")
    c0 = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    c1 = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    print(f"zk_gemm_f16_frag M={M} K={K} N={N}", flush=True)
    L.call("zk_gemm_f16", ta.data_ptr(), tw.data_ptr(), c0.data_ptr(), M, N, K, K, K, N, 1,
           L.ZK_F16, tb.data_ptr(), None, 0, L.ZK_EPI_BIAS, _stream())
    L.call("zk_gemm_f16_frag", af.data_ptr(), tw.data_ptr(), c1.data_ptr(), M, N, K, K, N,
           tb.data_ptr(), _stream())
    torch.cuda.synchronize()
    assert not torch.isnan(c1).any()
    if K >= 2048:
        assert torch.equal(c0.view(torch.int16), c1.view(torch.int16))
    else:
        ok, worst = fp16_tol(c1.float().cpu().numpy(), ops.linear(a, w, b))
        assert ok, worst

"""GPU parity: flash-attention forward (fp16 MFMA and fp32 paths) with the
key-padding mask, vs the float64 dense masked-softmax oracle.

fp16 bar: |O - ref| <= 2e-3 + 1e-2 |ref|; fp32 bar: 1e-5 abs + 1e-4 rel.
"""

import math

import numpy as np
import pytest
import torch

from oracle import ops
from tests.conftest import fp16_tol
from zenith_amd import synthetic

pytestmark = pytest.mark.gpu


def _qkv(B, H, Sq, Sk, D, f16=True, tag=0):
    q = synthetic.normal((B, H, Sq, D), tag=tag + 1)
    k = synthetic.normal((B, H, Sk, D), tag=tag + 2)
    v = synthetic.normal((B, H, Sk, D), tag=tag + 3)
    if f16:
        q, k, v = (synthetic.round_f16(a) for a in (q, k, v))
    return q, k, v


def _run(dev, q, k, v, lens, dtype):
    from zenith_amd import zenith_cuda as zc

    t = [torch.from_numpy(a).to(dev, dtype) for a in (q, k, v)]
    tl = None if lens is None else torch.from_numpy(np.asarray(lens, np.int32)).to(dev)
    return zc.flash_attention(*t, key_padding_lengths=tl).float().cpu().numpy()


@pytest.mark.parametrize("B,H,S,D", [(2, 12, 128, 64), (2, 3, 512, 64), (3, 2, 77, 64),
                                     (2, 2, 130, 128), (2, 2, 64, 32), (1, 1, 1, 64),
                                     (2, 4, 300, 64), (4, 2, 100, 64), (3, 2, 400, 64),
                                     (2, 4, 777, 64), (2, 2, 600, 48)])
@pytest.mark.parametrize("masked", [False, True])
def test_flash_attention_f16(dev, B, H, S, D, masked):
    """B*H a multiple of 8 with 2 and 3 query blocks per head exercises the
    workgroup remap that puts the blocks of one head on one XCD; B*H = 6 or 4
    keeps the direct order."""
    q, k, v = _qkv(B, H, S, S, D)
    lens = None
    if masked:
        lens = np.random.default_rng(3).integers(S // 2, S, size=B, endpoint=True)
        lens[0] = max(1, S // 2)
    o = _run(dev, q, k, v, lens, torch.float16)
    ok, worst = fp16_tol(o, ops.attention(q, k, v, lens))
    assert ok, worst


@pytest.mark.parametrize("S", [128, 512])
def test_flash_attention_config3(dev, S):
    """Config 3: B=32, H=12, D=64, lengths ~ U{S/2..S}; every one of the 32
    sequences against the float64 oracle."""
    B, H, D = 32, 12, 64
    q, k, v = _qkv(B, H, S, S, D, tag=10)
    lens = synthetic.padding_lengths(B, S)
    o = _run(dev, q, k, v, lens, torch.float16)
    for lo in range(0, B, 8):
        sl = slice(lo, lo + 8)
        ok, worst = fp16_tol(o[sl], ops.attention(q[sl], k[sl], v[sl], lens[sl]))
        assert ok, (lo, worst)


@pytest.mark.parametrize("S", [128, 512])
def test_flash_attention_config3_batch_invariance(dev, S):
    """Each of the 32 sequences run alone (B=1, where the workgroup remap of
    B*H % 8 == 0 grids is off) is bit-identical to its row of the B=32
    launch: the arithmetic of a (batch, head) does not depend on where its
    workgroups land, so any batch-indexing error shows as a mismatch."""
    from zenith_amd import zenith_cuda as zc

    B, H, D = 32, 12, 64
    q, k, v = (torch.from_numpy(a).to(dev, torch.float16) for a in _qkv(B, H, S, S, D, tag=10))
    lens = torch.from_numpy(synthetic.padding_lengths(B, S)).to(dev)
    full = zc.flash_attention(q, k, v, key_padding_lengths=lens)
    for b in range(B):
        one = zc.flash_attention(q[b:b + 1], k[b:b + 1], v[b:b + 1],
                                 key_padding_lengths=lens[b:b + 1])
        assert torch.equal(one, full[b:b + 1]), b


@pytest.mark.parametrize("D", [8, 24, 40, 48, 56, 72, 80, 96, 112, 120])
@pytest.mark.parametrize("S", [77, 128, 300])
def test_flash_attention_f16_any_head_dim(dev, D, S):
    """head_dim below the compiled widths 32 / 64 / 128 (zero-padded inside
    the kernel), masked, ragged lengths."""
    B, H = 3, 2
    q, k, v = _qkv(B, H, S, S, D, tag=100 + D)
    lens = np.array([S, S // 2 + 1, 1], np.int32)
    o = _run(dev, q, k, v, lens, torch.float16)
    assert o.shape == (B, H, S, D)
    ok, worst = fp16_tol(o, ops.attention(q, k, v, lens))
    assert ok, worst


@pytest.mark.parametrize("D", [5, 20, 33, 100])
def test_flash_attention_f16_odd_head_dim(dev, D):
    """fp16 head_dims that are not a multiple of 8: padded to one by the
    Python layer, scale still 1/sqrt(D)."""
    q, k, v = _qkv(2, 3, 70, 70, D, tag=120 + D)
    lens = np.array([70, 40], np.int32)
    o = _run(dev, q, k, v, lens, torch.float16)
    assert o.shape == (2, 3, 70, D)
    ok, worst = fp16_tol(o, ops.attention(q, k, v, lens))
    assert ok, worst


def _mask_case(kind, B, H, S, rng):
    """Boolean masks (True = attend) in the broadcast forms SDPA accepts."""
    if kind == "hf_padding":  # HF BERT's SDPA mask: [B, 1, S, S], rows equal
        lens = rng.integers(1, S + 1, size=B)
        keep = np.arange(S)[None, :] < lens[:, None]
        return np.broadcast_to(keep[:, None, None, :], (B, 1, S, S)).copy()
    if kind == "keys_only":  # [B, 1, 1, S], not a prefix
        return rng.random((B, 1, 1, S)) < 0.7
    if kind == "per_query":  # [B, H, S, S] with some rows fully masked
        m = rng.random((B, H, S, S)) < 0.5
        m[0, 0, :3, :] = False
        m[-1, -1, -1, :] = False
        return m
    if kind == "shared_2d":  # [S, S], broadcast over batch and heads
        return rng.random((S, S)) < 0.8
    raise ValueError(kind)


@pytest.mark.parametrize("B,H,S,D", [(2, 3, 128, 64), (2, 2, 300, 64), (2, 2, 77, 48),
                                     (1, 2, 130, 128), (2, 2, 64, 32), (1, 2, 520, 64)])
@pytest.mark.parametrize("kind", ["hf_padding", "keys_only", "per_query", "shared_2d"])
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_flash_attention_bool_mask(dev, B, H, S, D, kind, dtype):
    """Boolean attn_mask on the 16-query kernel (S <= 128, D = 64), the
    32-query kernel, the zero-padded head_dim kernel and fp32, combined with
    key-padding lengths; rows with no key left give 0. S = 77 / 130 take the
    padded mask copy (keys not a multiple of 4)."""
    from zenith_amd import zenith_cuda as zc

    kinds = ["hf_padding", "keys_only", "per_query", "shared_2d"]
    rng = np.random.default_rng([B, H, S, D, kinds.index(kind)])
    q, k, v = _qkv(B, H, S, S, D, f16=dtype == "f16", tag=160)
    mask = _mask_case(kind, B, H, S, rng)
    lens = np.full(B, S, np.int32)
    lens[0] = max(1, S - 20)
    tdt = torch.float16 if dtype == "f16" else torch.float32
    t = [torch.from_numpy(a).to(dev, tdt) for a in (q, k, v)]
    o = zc.flash_attention(*t, key_padding_lengths=torch.from_numpy(lens).to(dev),
                           attn_mask=torch.from_numpy(mask).to(dev)).float().cpu().numpy()
    ref = ops.attention(q, k, v, lens, mask=mask)
    if dtype == "f16":
        ok, worst = fp16_tol(o, ref)
        assert ok, worst
    else:
        np.testing.assert_allclose(o, ref, rtol=1e-4, atol=1e-5)
    empty = ~np.broadcast_to(mask, (B, H, S, S)).any(-1)
    assert not o[empty].any()


def test_flash_attention_mask_matches_lengths(dev):
    """A prefix mask equal to the key-padding lengths gives the same output
    as the lengths alone, bit for bit (config 3 at s128 and a 32-query
    shape)."""
    from zenith_amd import zenith_cuda as zc

    for B, H, S in ((32, 12, 128), (4, 12, 512)):
        q, k, v = (torch.from_numpy(a).to(dev, torch.float16) for a in _qkv(B, H, S, S, 64, tag=170))
        lens = torch.from_numpy(synthetic.padding_lengths(B, S)).to(dev)
        keep = torch.arange(S, device=dev)[None, :] < lens[:, None]
        a = zc.flash_attention(q, k, v, key_padding_lengths=lens)
        b = zc.flash_attention(q, k, v, attn_mask=keep[:, None, None, :])
        assert torch.equal(a, b)


def test_flash_attention_mask_rejects_float_masks(dev):
    from zenith_amd import zenith_cuda as zc

    q = torch.zeros(1, 1, 8, 64, device=dev, dtype=torch.float16)
    with pytest.raises(RuntimeError):
        zc.flash_attention(q, q, q, attn_mask=torch.zeros(8, 8, device=dev))


@pytest.mark.parametrize("D", [1, 17, 48, 80, 96, 127])
def test_flash_attention_f32_any_head_dim(dev, D):
    q, k, v = _qkv(2, 2, 65, 65, D, f16=False, tag=140 + D)
    lens = np.array([65, 33], np.int32)
    o = _run(dev, q, k, v, lens, torch.float32)
    np.testing.assert_allclose(o, ops.attention(q, k, v, lens), rtol=1e-4, atol=1e-5)


def test_flash_attention_edge_lengths(dev):
    """Length 0 -> zero output; length 1 -> O = V[0]; length S -> unmasked."""
    B, H, S, D = 4, 2, 96, 64
    q, k, v = _qkv(B, H, S, S, D, tag=20)
    lens = np.array([0, 1, S, 65], np.int32)
    o = _run(dev, q, k, v, lens, torch.float16)
    assert np.all(o[0] == 0)
    np.testing.assert_allclose(o[1], np.broadcast_to(v[1, :, :1, :], o[1].shape), atol=2e-3, rtol=1e-2)
    ok, worst = fp16_tol(o, ops.attention(q, k, v, lens))
    assert ok, worst


def test_flash_attention_uniform_keys(dev):
    """Identical keys -> O = mean of the valid V rows (closed form)."""
    B, H, S, D = 2, 2, 128, 64
    q, _, v = _qkv(B, H, S, S, D, tag=30)
    k = np.broadcast_to(synthetic.round_f16(synthetic.normal((1, 1, 1, D), tag=33)), (B, H, S, D)).copy()
    lens = np.array([100, 37], np.int32)
    o = _run(dev, q, k, v, lens, torch.float16)
    for b in range(B):
        mean = v[b, :, : lens[b], :].astype(np.float64).mean(axis=1, keepdims=True)
        np.testing.assert_allclose(o[b], np.broadcast_to(mean, o[b].shape), atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("S,lens", [(128, [128, 70, 64]), (512, [512, 300, 65])])
def test_flash_attention_strided_qkv(dev, S, lens):
    """Q/K/V read by stride out of a packed [B*S, 3H] projection, O written
    into [B*S, H]: the layout the encoder uses (no transposes). At S = 512
    the K/V rows are 3H apart in the DMA ring kernel's buffer reads."""
    from zenith_amd import _lib as L

    B, nh, D = 3, 12, 64
    H = nh * D
    qkv = synthetic.round_f16(synthetic.normal((B * S, 3 * H), tag=40))
    lens = np.array(lens, np.int32)
    tq = torch.from_numpy(qkv).to(dev, torch.float16)
    out = torch.empty((B * S, H), dtype=torch.float16, device=dev)
    base, es = tq.data_ptr(), 2
    ld = 3 * H
    L.call("zk_flash_attn_fwd", base, base + H * es, base + 2 * H * es, out.data_ptr(), B, nh, S, S, D,
           L.strides_arg([S * ld, D, ld] * 3 + [S * H, D, H]),
           torch.from_numpy(lens).to(dev).data_ptr(), 1.0 / math.sqrt(D), L.ZK_F16,
           torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    x = qkv.reshape(B, S, 3, nh, D).transpose(2, 0, 3, 1, 4)  # 3,B,nh,S,D
    ref = ops.attention(x[0], x[1], x[2], lens).transpose(0, 2, 1, 3).reshape(B * S, H)
    ok, worst = fp16_tol(out.float().cpu().numpy(), ref)
    assert ok, worst


@pytest.mark.parametrize("B,H,S,D", [(2, 4, 128, 64), (1, 2, 77, 32), (2, 2, 65, 128)])
@pytest.mark.parametrize("masked", [False, True])
def test_flash_attention_f32(dev, B, H, S, D, masked):
    q, k, v = _qkv(B, H, S, S, D, f16=False, tag=50)
    lens = np.array([S // 2 + 1] + [S] * (B - 1), np.int32) if masked else None
    o = _run(dev, q, k, v, lens, torch.float32)
    np.testing.assert_allclose(o, ops.attention(q, k, v, lens), rtol=1e-4, atol=1e-5)


def test_flash_attention_cross_lengths(dev):
    """Sq != Sk."""
    q, _, _ = _qkv(2, 2, 40, 40, 64, tag=60)
    _, k, v = _qkv(2, 2, 200, 200, 64, tag=70)
    o = _run(dev, q, k, v, [150, 200], torch.float16)
    ok, worst = fp16_tol(o, ops.attention(q, k, v, np.array([150, 200])))
    assert ok, worst


@pytest.mark.parametrize("Sk,lens", [(200, [150, 200, 0, 1]), (130, [130, 65, 129, 64])])
def test_flash_attention_long_queries_ragged_keys(dev, Sk, lens):
    """Sq >= 128 with Sk not a multiple of the 64-key tile: the last tile's
    rows past Sk must read as zeros; lengths 0, 1, a tile boundary, Sk."""
    q, _, _ = _qkv(4, 3, 128, 128, 64, tag=80)
    _, k, v = _qkv(4, 3, Sk, Sk, 64, tag=85)
    lens = np.array(lens, np.int32)
    o = _run(dev, q, k, v, lens, torch.float16)
    assert np.all(o[lens == 0] == 0)
    ok, worst = fp16_tol(o, ops.attention(q, k, v, lens))
    assert ok, worst


@pytest.mark.parametrize("Sk,lens", [(450, [450, 0, 1, 64]), (200, [129, 200, 63, 2])])
def test_flash_attention_ring_ragged_keys(dev, Sk, lens):
    """From 384 queries (D = 64, lengths only) K and V reach LDS by DMA into a
    ring of tile stages: Sk not a multiple of the 64-key tile (rows past Sk
    read as zeros through the buffer bound), lengths 0, 1 and at tile
    boundaries, Sq != Sk in both directions."""
    q, _, _ = _qkv(4, 3, 400, 400, 64, tag=90)
    _, k, v = _qkv(4, 3, Sk, Sk, 64, tag=95)
    lens = np.array(lens, np.int32)
    o = _run(dev, q, k, v, lens, torch.float16)
    assert np.all(o[lens == 0] == 0)
    ok, worst = fp16_tol(o, ops.attention(q, k, v, lens))
    assert ok, worst


@pytest.mark.parametrize("S", [128, 512])
def test_flash_attention_deterministic(dev, S):
    """Repeated launches on the same inputs give bit-identical outputs (the
    kernel has no atomics or reduction-order freedom; a difference means a
    read racing a write or a missing wait on a matrix-core result)."""
    from zenith_amd import zenith_cuda as zc

    B, H, D = 8, 12, 64
    q, k, v = (torch.from_numpy(a).to(dev, torch.float16) for a in _qkv(B, H, S, S, D, tag=90))
    lens = torch.from_numpy(synthetic.padding_lengths(B, S, seed=9)).to(dev)
    first = zc.flash_attention(q, k, v, key_padding_lengths=lens)
    for _ in range(5):
        again = zc.flash_attention(q, k, v, key_padding_lengths=lens)
        assert torch.equal(again, first)

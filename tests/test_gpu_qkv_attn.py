"""GPU parity: fused QKV projection + attention (zk_qkv_attn_f16), sequences
of 64 and 128 tokens, head_dim 64, weights interleaved per head (q_h, k_h,
v_h rows).

Oracle: qkv = x . W^T + b in float32, rounded to fp16 (what the unfused GEMM
stores), then the float64 masked-softmax attention per (sequence, head);
fp16 bar |y - ref| <= 2e-3 + 1e-2 |ref|. Also checked against the unfused
C-ABI pair (zk_gemm_f16 with the bias epilogue, then zk_flash_attn_fwd
reading the per-head column blocks by stride) at the same bar, and for
bit-exact batch invariance: every sequence run alone must equal its rows of
the batched launch (a tile's Q, K, V and a sequence's attention do not depend
on the other sequences, whatever tile the sequence lands in).
"""

import math

import numpy as np
import pytest
import torch

from oracle import ops
from tests.conftest import fp16_tol
from zenith_amd import _lib as L
from zenith_amd import synthetic

pytestmark = pytest.mark.gpu

D = 64


def _inputs(B, S, heads, tag=0):
    H = heads * D
    x = synthetic.round_f16(synthetic.normal((B * S, H), tag=60 + tag))
    w = synthetic.round_f16(synthetic.normal((3 * H, H), tag=61 + tag, std=0.05))
    b = synthetic.round_f16(synthetic.normal((3 * H,), tag=62 + tag, std=0.1))
    return x, w, b


def _lens(B, S, seed=0):
    """Lengths ~ U{1..S} with the edge values 0, 1, 63, 64, 65 and S first."""
    lens = np.random.default_rng([B, S, seed]).integers(1, S, size=B, endpoint=True)
    edges = [v for v in (0, 1, 63, 64, 65, S) if v <= S]
    lens[:min(B, len(edges))] = edges[:B]
    return lens.astype(np.int32)


def _oracle(x, w, b, lens, B, S, heads):
    qkv = synthetic.round_f16(ops.linear(x, w, b)).reshape(B, S, heads, 3, D)
    q, k, v = (np.ascontiguousarray(qkv[:, :, :, i].transpose(0, 2, 1, 3)) for i in range(3))
    o = ops.attention(q, k, v, lens)  # [B, heads, S, D]
    return o.transpose(0, 2, 1, 3).reshape(B * S, heads * D)


def _fused(dev, x, w, b, lens, B, S, heads):
    H = heads * D
    tx, tw, tb = (torch.from_numpy(a).to(dev, torch.float16) for a in (x, w, b))
    ctx = torch.full((B * S, H), float("nan"), dtype=torch.float16, device=dev)
    tl = None if lens is None else torch.from_numpy(lens).to(dev)
    print(f"zk_qkv_attn_f16 B={B} S={S} heads={heads}", flush=True)
    L.call("zk_qkv_attn_f16", tx.data_ptr(), tw.data_ptr(), tb.data_ptr(), ctx.data_ptr(),
           B, S, H, heads, None if tl is None else tl.data_ptr(), 1.0 / math.sqrt(D),
           torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return ctx.float().cpu().numpy()


def _unfused(dev, x, w, b, lens, B, S, heads):
    H = heads * D
    s = torch.cuda.current_stream().cuda_stream
    tx, tw, tb = (torch.from_numpy(a).to(dev, torch.float16) for a in (x, w, b))
    qkv = torch.empty((B * S, 3 * H), dtype=torch.float16, device=dev)
    ctx = torch.empty((B * S, H), dtype=torch.float16, device=dev)
    L.call("zk_gemm_f16", tx.data_ptr(), tw.data_ptr(), qkv.data_ptr(), B * S, 3 * H, H, H, H,
           3 * H, 1, L.ZK_F16, tb.data_ptr(), None, 0, L.ZK_EPI_BIAS, s)
    ld = 3 * H
    st = L.strides_arg([S * ld, 3 * D, ld, S * ld, 3 * D, ld, S * ld, 3 * D, ld, S * H, D, H])
    tl = None if lens is None else torch.from_numpy(lens).to(dev)
    base, es = qkv.data_ptr(), qkv.element_size()
    L.call("zk_flash_attn_fwd", base, base + D * es, base + 2 * D * es, ctx.data_ptr(), B, heads,
           S, S, D, st, None if tl is None else tl.data_ptr(), 1.0 / math.sqrt(D), L.ZK_F16, s)
    torch.cuda.synchronize()
    return ctx.float().cpu().numpy()


@pytest.mark.parametrize("B,S,heads", [(32, 128, 12), (3, 128, 12), (5, 64, 4), (1, 128, 2),
                                       (8, 64, 12), (7, 64, 3)])
@pytest.mark.parametrize("masked", [True, False])
def test_qkv_attn_vs_oracle(dev, B, S, heads, masked):
    """Config-5 shape (b32 s128, 12 heads) and ragged batches: an odd number
    of 128-token sequences or of 64-token ones leaves the last 256-row tile
    partly empty."""
    x, w, b = _inputs(B, S, heads)
    lens = _lens(B, S) if masked else None
    y = _fused(dev, x, w, b, lens, B, S, heads)
    ok, worst = fp16_tol(y, _oracle(x, w, b, lens, B, S, heads))
    assert ok, worst


@pytest.mark.parametrize("B,S,heads", [(32, 128, 12), (6, 64, 4)])
def test_qkv_attn_vs_unfused(dev, B, S, heads):
    x, w, b = _inputs(B, S, heads, tag=5)
    lens = _lens(B, S, seed=1)
    y = _fused(dev, x, w, b, lens, B, S, heads)
    ok, worst = fp16_tol(y, _unfused(dev, x, w, b, lens, B, S, heads))
    assert ok, worst


@pytest.mark.parametrize("S", [128, 64])
def test_qkv_attn_batch_invariance(dev, S):
    B, heads = 8, 12
    x, w, b = _inputs(B, S, heads, tag=9)
    lens = _lens(B, S, seed=2)
    y = _fused(dev, x, w, b, lens, B, S, heads)
    for i in range(B):
        yi = _fused(dev, x[i * S:(i + 1) * S], w, b, lens[i:i + 1], 1, S, heads)
        np.testing.assert_array_equal(yi, y[i * S:(i + 1) * S])


def test_qkv_attn_zero_length_rows_are_zero(dev):
    """A sequence with no valid key produces 0, as in zk_flash_attn_fwd."""
    B, S, heads = 2, 128, 2
    x, w, b = _inputs(B, S, heads, tag=11)
    lens = np.array([0, S], np.int32)
    y = _fused(dev, x, w, b, lens, B, S, heads)
    assert np.all(y[:S] == 0)
    assert np.all(np.isfinite(y[S:]))

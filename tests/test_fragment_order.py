"""Host side of the fragment-ordered FFN intermediate: to_fragment_order and
from_fragment_order (encoder.py) against the layout's definitions in
include/zk_api.h (fp16: 16 columns per k-step; int8: 32), element by element
on a ragged shape, and the round trip. CPU only (torch on the host)."""

import torch

from zenith_amd.encoder import from_fragment_order, to_fragment_order


def test_fragment_order_layout():
    R, K = 70, 48
    x = (torch.arange(R * K) % 2000).to(torch.float16).reshape(R, K)
    p = to_fragment_order(x)
    Rp = 96
    assert p.numel() == Rp * K
    for m in range(Rp):
        for k in range(K):
            rb, ks = m // 32, k // 16
            lane = m % 32 + 32 * ((k % 16) // 8)
            v = p[(rb * (K // 16) + ks) * 512 + 8 * lane + k % 8]
            assert v == (x[m, k] if m < R else 0), (m, k)
    assert torch.equal(from_fragment_order(p, R, K), x)


def test_fragment_order_layout_int8():
    R, K = 45, 96
    x = (torch.arange(R * K) % 251 - 125).to(torch.int8).reshape(R, K)
    p = to_fragment_order(x)
    Rp = 64
    assert p.numel() == Rp * K and p.dtype == torch.int8
    for m in range(Rp):
        for k in range(K):
            rb, ks = m // 32, k // 32
            lane = m % 32 + 32 * ((k % 32) // 16)
            v = p[(rb * (K // 32) + ks) * 1024 + 16 * lane + k % 16]
            assert v == (x[m, k] if m < R else 0), (m, k)
    assert torch.equal(from_fragment_order(p, R, K), x)

"""Host side of the fragment-ordered FFN intermediate: to_fragment_order and
from_fragment_order (encoder.py) against the layout's definition in
include/zk_api.h, element by element on a ragged shape, and the round trip.
CPU only (torch on the host)."""

import torch

from zenith_amd.encoder import from_fragment_order, to_fragment_order


def test_fragment_order_layout():
    R, K = 70, 48
    x = torch.arange(R * K, dtype=torch.float32).reshape(R, K)
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

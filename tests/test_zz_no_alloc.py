"""GPU: zk_gemm_f16_noalloc (split-K partials in the library's static device
array) against zk_gemm_f16_ws (partials in a torch-allocated workspace), both
through the C ABI. Same kernels and the same split plan, so the outputs must
be bit-identical; two split calls in a row (the second smaller, so the array
still holds the first call's partials) and one unsplit call."""

import numpy as np
import pytest
import torch

from oracle import ops
from tests.conftest import fp16_tol
from zenith_amd import _lib as L
from zenith_amd import synthetic

pytestmark = pytest.mark.gpu


def _gemm_pair(dev, M, K, N, epi, tag):
    lib = L.load()
    x = synthetic.round_f16(synthetic.normal((M, K), tag=tag))
    w = synthetic.round_f16(synthetic.normal((N, K), tag=tag + 1, std=0.05))
    b = synthetic.round_f16(synthetic.normal((N,), tag=tag + 2, std=0.5))
    tx, tw, tb = (torch.from_numpy(a).to(dev, torch.float16) for a in (x, w, b))
    need = int(lib.zk_gemm_workspace_size(M, N, K, L.ZK_F16))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    c_ws = torch.empty((M, N), dtype=torch.float16, device=dev)
    c_na = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    L.call("zk_gemm_f16_ws", tx.data_ptr(), tw.data_ptr(), c_ws.data_ptr(), M, N, K, K, K, N, 1,
           L.ZK_F16, tb.data_ptr(), None, 0, epi, ws.data_ptr(), need, s)
    L.call("zk_gemm_f16_noalloc", tx.data_ptr(), tw.data_ptr(), c_na.data_ptr(), M, N, K, K, K,
           N, 1, L.ZK_F16, tb.data_ptr(), None, 0, epi, s)
    torch.cuda.synchronize()
    return need, c_ws, c_na, x, w, b


def test_noalloc_matches_workspace_entry_point(dev):
    cases = [(512, 3072, 768, L.ZK_EPI_BIAS, 50),          # 4 splits, 6 MiB of partials
             (128, 3072, 768, L.ZK_EPI_BIAS, 10),          # smaller: 10 splits, 3.75 MiB
             (64, 768, 768, L.ZK_EPI_BIAS_GELU_ERF, 20),   # smaller: 6 splits
             (4096, 768, 3072, L.ZK_EPI_BIAS, 30)]         # not split: no scratch used
    for M, K, N, epi, tag in cases:
        need, c_ws, c_na, x, w, b = _gemm_pair(dev, M, K, N, epi, tag)
        print(f"noalloc M={M} K={K} N={N} epi={epi}: partials {need} bytes", flush=True)
        assert (need > 0) == (M < 4096)
        assert need <= 8 << 20
        assert torch.equal(c_na, c_ws), (M, K, N)
        ref = ops.matmul_f64(x, w.T) + b
        if epi == L.ZK_EPI_BIAS_GELU_ERF:
            ref = ops.gelu_erf(ref.astype(np.float32))
        ok, worst = fp16_tol(c_na.float().cpu().numpy(), ref)
        assert ok, worst


def test_noalloc_argument_errors_match(dev):
    """Bad arguments fail with the same status as zk_gemm_f16, before any
    launch (no scratch lookup needed)."""
    lib = L.load()
    for args in ((16, 16, 16, 8, 8, 12, 12, 12, 8, 1, L.ZK_F16, None, None, 0, 0, None),
                 (16, 16, 16, 8, 8, 8, 4, 8, 8, 1, L.ZK_F16, None, None, 0, 0, None)):
        assert lib.zk_gemm_f16_noalloc(*args) == lib.zk_gemm_f16(*args) != 0


def test_noalloc_under_graph_capture(dev):
    """A split-K call captured into a HIP graph (torch.cuda.CUDAGraph) and
    replayed: every replay is bit-identical to zk_gemm_f16_ws, also after an
    eager call of another shape has overwritten the static array between
    replays (each split writes its whole partial tile before the reduction
    reads it, so nothing has to be cleared). The first call on a device
    looks the array's device address up, which is done here eagerly, before
    capture, as the header asks; after it a call makes no HIP API call
    besides its two launches."""
    lib = L.load()
    M, K, N = 128, 3072, 768
    need, c_ws, c_na, x, w, b = _gemm_pair(dev, M, K, N, L.ZK_EPI_BIAS, 40)
    assert need > 0 and torch.equal(c_na, c_ws)
    tx, tw, tb = (torch.from_numpy(a).to(dev, torch.float16) for a in (x, w, b))
    out = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st = lib.zk_gemm_f16_noalloc(tx.data_ptr(), tw.data_ptr(), out.data_ptr(), M, N, K, K, K,
                                     N, 1, L.ZK_F16, tb.data_ptr(), None, 0, L.ZK_EPI_BIAS,
                                     torch.cuda.current_stream().cuda_stream)
    assert st == 0, L.last_error()
    for i in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, c_ws), f"replay {i}"
        # eager work between replays: a smaller split call on the same array
        _, s_ws, s_na, *_ = _gemm_pair(dev, 64, 768, 768, L.ZK_EPI_BIAS_GELU_ERF, 50 + i)
        assert torch.equal(s_na, s_ws)

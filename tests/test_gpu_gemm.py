"""GPU parity: FP16 MFMA GEMM (wmma_matmul / linear with fused epilogues) and
the fp32 `matmul`, vs the CPU oracle.

FP16 GEMM bar: |C - ref| <= 2e-3 + 1e-2 |ref| with ref the float64 product of
the same fp16-rounded inputs (every product is exact in float64). Large
squares are checked on a seeded sample of rows (rows are independent).
"""

import numpy as np
import pytest
import torch

from oracle import ops
from tests.conftest import fp16_tol
from zenith_amd import synthetic

pytestmark = pytest.mark.gpu

BERT = [(4096, 768, 2304), (4096, 768, 768), (4096, 768, 3072), (4096, 3072, 768)]


def _t(a, dev, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev, dtype)


@pytest.mark.parametrize("M,K,N", [(128, 64, 256), (64, 64, 64), (100, 70, 37), (1, 8, 1),
                                   (257, 136, 129), (1024, 1024, 1024)] + BERT)
@pytest.mark.parametrize("out", [torch.float32, torch.float16])
def test_wmma_matmul(dev, M, K, N, out):
    from zenith_amd import zenith_cuda as zc

    a = synthetic.round_f16(synthetic.uniform((M, K), tag=1))
    b = synthetic.round_f16(synthetic.uniform((K, N), tag=2))
    c = zc.wmma_matmul(_t(a, dev, torch.float16), _t(b, dev, torch.float16), out_dtype=out)
    assert c.dtype == out and c.shape == (M, N)
    ref = ops.matmul_f64(a, b)
    ok, worst = fp16_tol(c.float().cpu().numpy(), ref)
    assert ok, worst


@pytest.mark.parametrize("n", [4096, 8192])
def test_wmma_matmul_square_sampled(dev, n):
    from zenith_amd import zenith_cuda as zc

    a = synthetic.round_f16(synthetic.uniform((n, n), tag=3))
    b = synthetic.round_f16(synthetic.uniform((n, n), tag=4))
    c = zc.wmma_matmul(_t(a, dev, torch.float16), _t(b, dev, torch.float16), out_dtype=torch.float16)
    rows = np.random.default_rng(7).choice(n, 48, replace=False)
    ref = ops.matmul_f64(a[rows], b)
    ok, worst = fp16_tol(c[torch.from_numpy(rows).to(dev)].float().cpu().numpy(), ref)
    assert ok, worst


def test_wmma_matmul_reference_kat(dev):
    """[[1,2,3],[4,5,6]] . [[1,2],[3,4],[5,6]] = [[22,28],[49,64]]
    (tests/test_kernels.cpp:68-86)."""
    from zenith_amd import zenith_cuda as zc

    a = torch.tensor([[1, 2, 3], [4, 5, 6]], dtype=torch.float16, device=dev)
    b = torch.tensor([[1, 2], [3, 4], [5, 6]], dtype=torch.float16, device=dev)
    np.testing.assert_array_equal(zc.wmma_matmul(a, b).cpu().numpy(), [[22, 28], [49, 64]])
    np.testing.assert_array_equal(zc.matmul(a.float(), b.float()).cpu().numpy(), [[22, 28], [49, 64]])


@pytest.mark.parametrize("act", [None, "gelu", "gelu_tanh", "relu", "residual"])
@pytest.mark.parametrize("M,K,N", [(4096, 768, 3072), (4096, 3072, 768), (300, 768, 2304), (5, 24, 40)])
def test_linear_epilogues(dev, act, M, K, N):
    from zenith_amd import zenith_cuda as zc

    x = synthetic.round_f16(synthetic.normal((M, K), tag=5))
    w = synthetic.round_f16(synthetic.normal((N, K), tag=6, std=0.02))
    b = synthetic.round_f16(synthetic.normal((N,), tag=7, std=0.5))
    r = synthetic.round_f16(synthetic.normal((M, N), tag=8))
    y = zc.linear(_t(x, dev, torch.float16), _t(w, dev, torch.float16), _t(b, dev, torch.float16),
                  activation=None if act == "residual" else act,
                  residual=_t(r, dev, torch.float16) if act == "residual" else None)
    ref = ops.matmul_f64(x, w.T) + b
    if act == "gelu":
        ref = ops.gelu_erf(ref.astype(np.float32))
    elif act == "gelu_tanh":
        ref = ops.gelu_tanh(ref.astype(np.float32))
    elif act == "relu":
        ref = np.maximum(ref, 0)
    elif act == "residual":
        ref = ref + r
    ok, worst = fp16_tol(y.float().cpu().numpy(), ref)
    assert ok, worst


@pytest.mark.parametrize("M,K,N", [
    (4100, 72, 4100),   # 8-wave 256x256 tile, ragged M / N / K, scalar stores
    (4000, 100, 2000),  # 8-wave 256x192 tile, vector stores
    (520, 200, 20500),  # 128x128, 2-stage ring
    (700, 136, 1100),   # 128x96, 16x16 MFMA
    (1000, 3000, 600),  # 128x96, 4x1 waves, 3-stage ring (long K)
    (333, 500, 1000),   # 64x64, 16x16 MFMA
])
def test_linear_tile_configs(dev, M, K, N):
    """Every tile configuration of the shape-driven choice, at ragged edges,
    with the bias + residual epilogue."""
    from zenith_amd import zenith_cuda as zc

    x = synthetic.round_f16(synthetic.normal((M, K), tag=16))
    w = synthetic.round_f16(synthetic.normal((N, K), tag=17, std=0.05))
    b = synthetic.round_f16(synthetic.normal((N,), tag=18, std=0.5))
    r = synthetic.round_f16(synthetic.normal((M, N), tag=19))
    y = zc.linear(_t(x, dev, torch.float16), _t(w, dev, torch.float16), _t(b, dev, torch.float16),
                  residual=_t(r, dev, torch.float16))
    rows = np.random.default_rng(M).choice(M, min(M, 256), replace=False)
    rows.sort()
    ref = ops.matmul_f64(x[rows], w.T) + b + r[rows]
    got = y[torch.from_numpy(rows).to(dev)].float().cpu().numpy()
    ok, worst = fp16_tol(got, ref)
    assert ok, worst
    # edge rows and columns in full
    last = ops.matmul_f64(x[-3:], w.T) + b + r[-3:]
    ok, worst = fp16_tol(y[-3:].float().cpu().numpy(), last)
    assert ok, worst


def test_linear_3d_and_no_bias(dev):
    from zenith_amd import zenith_cuda as zc

    x = synthetic.round_f16(synthetic.normal((4, 33, 768), tag=9))
    w = synthetic.round_f16(synthetic.normal((768, 768), tag=10, std=0.02))
    y = zc.linear(_t(x, dev, torch.float16), _t(w, dev, torch.float16))
    assert y.shape == (4, 33, 768)
    ok, worst = fp16_tol(y.float().cpu().numpy(), ops.matmul_f64(x, w.T))
    assert ok, worst


@pytest.mark.parametrize("M,K,N", [(2, 3, 2), (128, 768, 768), (100, 70, 37), (513, 1000, 65)])
def test_matmul_fp32(dev, M, K, N):
    from zenith_amd import zenith_cuda as zc

    a = synthetic.uniform((M, K), tag=11)
    b = synthetic.uniform((K, N), tag=12)
    c = zc.matmul(_t(a, dev, torch.float32), _t(b, dev, torch.float32))
    assert c.dtype == torch.float32
    np.testing.assert_allclose(c.cpu().numpy(), ops.matmul_f64(a, b), rtol=1e-5, atol=1e-4)


def test_matmul_fp32_strided_b(dev):
    """B[K,N] read through a row stride wider than N (a column slice): the
    transpose + fp32 MFMA route (K % 4 == 0, large enough) copies it dense
    first; the SIMT route reads it by stride."""
    from zenith_amd import zenith_cuda as zc

    for M, K, N in ((256, 512, 384), (9, 10, 11)):
        a = synthetic.uniform((M, K), tag=13)
        big = synthetic.uniform((K, N + 12), tag=14)
        tb = _t(big, dev, torch.float32)[:, 5:5 + N]
        c = zc.matmul(_t(a, dev, torch.float32), tb)
        np.testing.assert_allclose(c.cpu().numpy(), ops.matmul_f64(a, big[:, 5:5 + N]),
                                   rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("M,K,N", [(256, 512, 384), (9, 10, 11), (64, 3, 33)])
def test_matmul_broadcast_operands(dev, M, K, N):
    """Broadcast views (expand(): stride(0) == 0) hold one row in memory; the
    product must read that row for every output row, never M rows of it (a
    past-the-allocation read). fp32 (transpose + MFMA route and SIMT route)
    and fp16 wmma_matmul."""
    from zenith_amd import zenith_cuda as zc

    x = synthetic.uniform((1, K), tag=15)
    y = synthetic.uniform((1, N), tag=16)
    ref = ops.matmul_f64(np.broadcast_to(x, (M, K)), np.broadcast_to(y, (K, N)))
    ta = _t(x, dev, torch.float32).expand(M, K)
    tb = _t(y, dev, torch.float32).expand(K, N)
    assert ta.stride(0) == 0 and tb.stride(0) == 0
    c = zc.matmul(ta, tb)
    np.testing.assert_allclose(c.cpu().numpy(), ref, rtol=1e-5, atol=1e-4)
    x16, y16 = synthetic.round_f16(x), synthetic.round_f16(y)
    c16 = zc.wmma_matmul(_t(x16, dev, torch.float16).expand(M, K),
                         _t(y16, dev, torch.float16).expand(K, N))
    ok, worst = fp16_tol(c16.cpu().numpy(), ops.matmul_f64(np.broadcast_to(x16, (M, K)),
                                                           np.broadcast_to(y16, (K, N))))
    assert ok, worst


@pytest.mark.parametrize("M,K,N", [
    (4100, 72, 4100),   # 8-wave 256x256 tile
    (4000, 100, 2000),  # 8-wave 256x192 tile
    (520, 200, 20500),  # 128x128, 2-stage ring
    (700, 136, 1100),   # 128x96, 16x16x4 fp32 MFMA
    (1000, 3000, 600),  # 128x96, 4x1 waves, 3-stage ring
    (333, 500, 1000),   # 64x64
    (128, 768, 3072),   # the hybrid encoder's FFN-up shape
    (77, 70, 33),       # K % 4 != 0: the SIMT kernel
])
def test_linear_fp32_tile_configs(dev, M, K, N):
    """fp32 Linear through the fp32-MFMA GEMM (every tile configuration, at
    ragged edges) and the SIMT fallback, vs the float64 product."""
    from zenith_amd import zenith_cuda as zc

    x = synthetic.normal((M, K), tag=40)
    w = synthetic.normal((N, K), tag=41, std=0.05)
    b = synthetic.normal((N,), tag=42)
    y = zc.linear(_t(x, dev, torch.float32), _t(w, dev, torch.float32), _t(b, dev, torch.float32))
    rows = np.random.default_rng(M).choice(M, min(M, 256), replace=False)
    rows.sort()
    ref = ops.matmul_f64(x[rows], w.T) + b
    got = y[torch.from_numpy(rows).to(dev)].cpu().numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(y[-2:].cpu().numpy(), ops.matmul_f64(x[-2:], w.T) + b, rtol=1e-4, atol=1e-4)


def test_linear_fp32(dev):
    from zenith_amd import zenith_cuda as zc

    x = synthetic.normal((64, 768), tag=13)
    w = synthetic.normal((3072, 768), tag=14, std=0.02)
    b = synthetic.normal((3072,), tag=15)
    y = zc.linear(_t(x, dev, torch.float32), _t(w, dev, torch.float32), _t(b, dev, torch.float32),
                  activation="gelu")
    np.testing.assert_allclose(y.cpu().numpy(), ops.gelu_erf(ops.linear(x, w, b)), rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("M,K,N", [(128, 3072, 768), (128, 768, 768), (37, 1000, 200), (128, 768, 3072),
                                   (64, 4096, 64), (64, 1152, 64), (64, 2304, 64)])
@pytest.mark.parametrize("act", [None, "gelu", "residual"])
def test_linear_split_k(dev, M, K, N, act):
    """Small-M products take the split-K path (caller workspace, fp32
    partials, ordered reduction with the epilogue): fp16 and fp32, against
    the float64 product, and bit-identical on repeated calls. The reduction
    reads its partials eight splits at a time: the last three shapes split
    16 ways (two whole groups), 9 and 12 ways in fp16 and 12 and 15 in fp32
    (a last group of 1 to 7)."""
    from zenith_amd import _lib as L
    from zenith_amd import zenith_cuda as zc

    assert L.load().zk_gemm_workspace_size(M, N, K, L.ZK_F32) > 0
    x = synthetic.normal((M, K), tag=50)
    w = synthetic.normal((N, K), tag=51, std=0.03)
    b = synthetic.normal((N,), tag=52, std=0.5)
    r = synthetic.normal((M, N), tag=53)
    ref = ops.matmul_f64(x, w.T) + b
    if act == "gelu":
        ref = ops.gelu_erf(ref.astype(np.float32))
    elif act == "residual":
        ref = ref + r
    kw = dict(activation="gelu" if act == "gelu" else None)
    y32 = zc.linear(_t(x, dev, torch.float32), _t(w, dev, torch.float32), _t(b, dev, torch.float32),
                    residual=_t(r, dev, torch.float32) if act == "residual" else None, **kw)
    np.testing.assert_allclose(y32.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)
    x16, w16, b16, r16 = (synthetic.round_f16(a) for a in (x, w, b, r))
    ref16 = ops.matmul_f64(x16, w16.T) + b16
    if act == "gelu":
        ref16 = ops.gelu_erf(ref16.astype(np.float32))
    elif act == "residual":
        ref16 = ref16 + r16
    args = (_t(x16, dev, torch.float16), _t(w16, dev, torch.float16), _t(b16, dev, torch.float16))
    res = _t(r16, dev, torch.float16) if act == "residual" else None
    y16 = zc.linear(*args, residual=res, **kw)
    ok, worst = fp16_tol(y16.float().cpu().numpy(), ref16)
    assert ok, worst
    for _ in range(3):
        assert torch.equal(zc.linear(*args, residual=res, **kw), y16)


@pytest.mark.parametrize("M,K,N", [(128, 256, 192), (37, 70, 29), (16, 768, 768), (300, 768, 3072)])
@pytest.mark.parametrize("epi", ["none", "bias", "gelu_erf", "gelu_tanh", "relu", "residual"])
def test_linear_f32_c_abi(dev, M, K, N, epi):
    """zk_linear_f32 through the C ABI on the three fp32 paths: the MFMA
    kernel (K % 4 == 0), the SIMT kernel with its separate epilogue pass
    (K = 70) and split-K with the epilogue in the ordered reduction (M = 16),
    each epilogue against the float64 product; rtol 1e-4 (fp32 products and
    accumulation; erf-GELU within 7.2e-7 absolute)."""
    from zenith_amd import _lib as L
    from zenith_amd.zenith_cuda import _ws_args, gemm_workspace

    x = synthetic.normal((M, K), tag=60)
    w = synthetic.normal((N, K), tag=61, std=0.05)
    b = synthetic.normal((N,), tag=62)
    r = synthetic.normal((M, N), tag=63)
    code = {"none": L.ZK_EPI_NONE, "bias": L.ZK_EPI_BIAS, "gelu_erf": L.ZK_EPI_BIAS_GELU_ERF,
            "gelu_tanh": L.ZK_EPI_BIAS_GELU_TANH, "relu": L.ZK_EPI_BIAS_RELU,
            "residual": L.ZK_EPI_BIAS_RESIDUAL}[epi]
    tx, tw, tb, tr = (_t(a, dev, torch.float32) for a in (x, w, b, r))
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    ws = gemm_workspace(M, N, K, L.ZK_F32, dev)
    L.call("zk_linear_f32", tx.data_ptr(), tw.data_ptr(), y.data_ptr(), M, N, K, K, K, N,
           None if epi == "none" else tb.data_ptr(), tr.data_ptr() if epi == "residual" else None,
           N, code, *_ws_args(ws), torch.cuda.current_stream().cuda_stream)
    ref = ops.matmul_f64(x, w.T)
    if epi != "none":
        ref = ref + b
    if epi == "gelu_erf":
        ref = ops.gelu_erf(ref.astype(np.float32))
    elif epi == "gelu_tanh":
        ref = ops.gelu_tanh(ref.astype(np.float32))
    elif epi == "relu":
        ref = ops.relu(ref)
    elif epi == "residual":
        ref = ref + r
    np.testing.assert_allclose(y.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("M,K,N,pad", [(128, 3072, 768, 192), (512, 3072, 768, 192),
                                       (128, 768, 768, 0), (512, 768, 768, 0),
                                       (256, 3072, 768, 192), (4096, 768, 768, 0),
                                       (96, 1000, 200, 24), (37, 3072, 96, 0),
                                       (320, 1024, 64, 8), (2048, 3072, 64, 0)])
def test_gemm_add_layernorm(dev, M, K, N, pad):
    """zk_gemm_f16_add_ln = the pair it replaces, bit for bit: zk_gemm_f16_ws
    (bias epilogue, fp16 out) into T, then zk_layernorm(T, R). Products that
    split along K take the fused path (the LayerNorm launch sums the split
    partials itself: four wavefronts per row below 2048 rows, one with at
    least 32 rows per split otherwise), the others the pair; both against the float64 product
    and the oracle's Add+LayerNorm at the fp16 bar. A and W with padded rows
    (the encoder's FFN intermediate), K not a multiple of the 128-byte slice
    (1000), N a multiple of 8 only (200, 96) and a ragged M (37)."""
    from zenith_amd import _lib as L

    lib = L.load()
    x = synthetic.round_f16(synthetic.normal((M, K), tag=60))
    w = synthetic.round_f16(synthetic.normal((N, K), tag=61, std=0.03))
    b = synthetic.round_f16(synthetic.normal((N,), tag=62, std=0.5))
    r = synthetic.round_f16(synthetic.normal((M, N), tag=63))
    g = synthetic.round_f16(1 + synthetic.normal((N,), tag=64, std=0.1))
    be = synthetic.round_f16(synthetic.normal((N,), tag=65, std=0.1))
    tx = torch.zeros((M, K + pad), dtype=torch.float16, device=dev)
    tx[:, :K] = _t(x, dev, torch.float16)
    tw = torch.zeros((N, K + pad), dtype=torch.float16, device=dev)
    tw[:, :K] = _t(w, dev, torch.float16)
    tb, tr, tg, tbe = (_t(a, dev, torch.float16) for a in (b, r, g, be))
    need = int(lib.zk_gemm_workspace_size(M, N, K, L.ZK_F16))
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    t_pair = torch.empty((M, N), dtype=torch.float16, device=dev)
    y_pair = torch.empty((M, N), dtype=torch.float16, device=dev)
    L.call("zk_gemm_f16_ws", tx.data_ptr(), tw.data_ptr(), t_pair.data_ptr(), M, N, K,
           tx.stride(0), tw.stride(0), N, 1, L.ZK_F16, tb.data_ptr(), None, 0, L.ZK_EPI_BIAS,
           ws.data_ptr(), need, s)
    L.call("zk_layernorm", t_pair.data_ptr(), tr.data_ptr(), tg.data_ptr(), tbe.data_ptr(),
           y_pair.data_ptr(), M, N, 1e-12, L.ZK_F16, s)
    t_buf = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    L.call("zk_gemm_f16_add_ln", tx.data_ptr(), tw.data_ptr(), tb.data_ptr(), tr.data_ptr(),
           tg.data_ptr(), tbe.data_ptr(), t_buf.data_ptr(), y.data_ptr(), M, N, K, tx.stride(0),
           tw.stride(0), 1e-12, ws.data_ptr(), need, s)
    torch.cuda.synchronize()
    # split products read the partials in the LayerNorm launch: four
    # wavefronts per row below 2048 rows of at most 1024 values, else one
    # wavefront per row with at least 32 rows per split
    splits = need // (M * N * 4)
    wide = M < 2048 and N <= 1024
    fused = need > 0 and (wide or splits * 32 <= M)
    assert torch.equal(y, y_pair), (M, K, N)
    if not fused:
        assert torch.equal(t_buf, t_pair)
    t_ref = synthetic.round_f16(ops.matmul_f64(x, w.T).astype(np.float32) + b)  # T is fp16
    ref = ops.add_layernorm(t_ref, r, g, be, 1e-12)
    ok, worst = fp16_tol(y.float().cpu().numpy(), ref)
    assert ok, worst
    kind = ("pair" if not fused else "partials, four wavefronts per row" if wide
            else "partials, one wavefront per row")
    print(f"gemm+add+LN M={M} K={K} N={N}: {kind}, "
          f"bit-identical to the pair", flush=True)

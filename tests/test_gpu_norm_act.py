"""GPU parity: LayerNorm / Add+LayerNorm, GELU / bias+GELU, ReLU, int8
quantisation — HIP kernels through the C ABI vs the CPU oracle.

Tolerances: fp32 I/O 1e-5 abs + 1e-5 rel (reference bar for LN is rtol 1e-4 /
atol 1e-5, tests/test_layernorm_parallel.py:45-79); fp16 outputs
|y - ref| <= 2e-3 + 1e-2 |ref| (north-star fp16 bar); quantisation bit-exact.
"""

import numpy as np
import pytest
import torch

from oracle import ops
from tests.conftest import fp16_tol
from zenith_amd import synthetic

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev, dtype)


@pytest.mark.parametrize("rows,hidden", [(1, 768), (128, 768), (4096, 768), (33, 1024),
                                         (7, 100), (5, 3), (16, 8192), (3, 20000),
                                         (8192, 768), (8200, 768)])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("with_res", [False, True])
def test_layernorm(dev, rows, hidden, dtype, with_res):
    """Rows of 768 fp16 values go two to a wavefront: 8192 rows are the
    largest launch that batches its loads (4096 wavefronts), 8200 the next
    shape, which loads one vector at a time."""
    from zenith_amd import zenith_cuda as zc

    x = synthetic.normal((rows, hidden), tag=1) * 3 + 0.5
    r = synthetic.normal((rows, hidden), tag=2)
    g = synthetic.normal((hidden,), tag=3, std=0.5) + 1
    b = synthetic.normal((hidden,), tag=4, std=0.1)
    eps = 1e-12 if hidden == 768 else 1e-5
    tdt = torch.float32 if dtype == "f32" else torch.float16
    if dtype == "f16":
        x, r, g, b = (synthetic.round_f16(a) for a in (x, r, g, b))
    if with_res:
        y = zc.add_layernorm(_t(x, dev, tdt), _t(r, dev, tdt), _t(g, dev, tdt), _t(b, dev, tdt), eps)
        ref = ops.add_layernorm(x, r, g, b, eps)
    else:
        y = zc.layernorm(_t(x, dev, tdt), _t(g, dev, tdt), _t(b, dev, tdt), eps)
        ref = ops.layernorm(x, g, b, eps)
    y = y.float().cpu().numpy()
    if dtype == "f32":
        np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)
    else:
        ok, worst = fp16_tol(y, ref)
        assert ok, worst


@pytest.mark.parametrize("rows,hidden", [(1, 768), (4096, 768), (33, 1024), (7, 100),
                                         (16, 8192)])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_layernorm_add(dev, rows, hidden, dtype):
    """LayerNormAdd: LN(x) * g + b + residual (the residual after the
    normalisation); hidden=100 takes the block-per-row kernel."""
    from zenith_amd import zenith_cuda as zc

    x = synthetic.normal((rows, hidden), tag=51) * 3 + 0.5
    r = synthetic.normal((rows, hidden), tag=52)
    g = synthetic.normal((hidden,), tag=53, std=0.5) + 1
    b = synthetic.normal((hidden,), tag=54, std=0.1)
    eps = 1e-12 if hidden == 768 else 1e-5
    tdt = torch.float32 if dtype == "f32" else torch.float16
    if dtype == "f16":
        x, r, g, b = (synthetic.round_f16(a) for a in (x, r, g, b))
    y = zc.layernorm_add(_t(x, dev, tdt), _t(r, dev, tdt), _t(g, dev, tdt), _t(b, dev, tdt), eps)
    y = y.float().cpu().numpy()
    ref = ops.layernorm_add(x, r, g, b, eps)
    if dtype == "f32":
        np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)
    else:
        ok, worst = fp16_tol(y, ref)
        assert ok, worst


def test_layernorm_add_through_the_registry(dev):
    """The GraphIR LayerNormAdd node, dispatched through the registry to the
    HIP kernel, in both node forms."""
    from zenith_amd.hooks.dispatcher import ExecutionContext, KernelDispatcher, Node
    from zenith_amd.hooks.kernel_registry import KernelRegistry, Precision

    reg = KernelRegistry()
    reg.initialize()
    d = KernelDispatcher(registry=reg, precision=Precision.FP16)
    x = synthetic.round_f16(synthetic.normal((64, 768), tag=55))
    r = synthetic.round_f16(synthetic.normal((64, 768), tag=56))
    g = synthetic.round_f16(synthetic.normal((768,), tag=57, std=0.3) + 1)
    b = synthetic.round_f16(synthetic.normal((768,), tag=58, std=0.1))
    T = lambda a: _t(a, dev, torch.float16)  # noqa: E731
    ctx = ExecutionContext({"x": T(x), "r": T(r), "g": T(g), "b": T(b)})
    y1 = d.dispatch(Node("LayerNormAdd", ["x", "r"], ["o"], {"epsilon": 1e-12}), ctx,
                    {"weight": T(g), "bias": T(b)})
    y2 = d.dispatch(Node("LayerNormAdd", ["x", "g", "b", "r"], ["o2"], {"epsilon": 1e-12}), ctx)
    assert torch.equal(y1, y2)
    ok, worst = fp16_tol(y1.float().cpu().numpy(), ops.layernorm_add(x, r, g, b, 1e-12))
    assert ok, worst


def test_layernorm_default_eps_and_unit_stats(dev):
    """layernorm(input, gamma, beta) uses eps=1e-5 like the reference
    binding; with gamma=1, beta=0 rows have mean 0 / std 1."""
    from zenith_amd import zenith_cuda as zc

    x = synthetic.normal((64, 768), tag=9) * 4 + 2
    y = zc.layernorm(_t(x, dev, torch.float32), torch.ones(768, device=dev),
                     torch.zeros(768, device=dev)).cpu().numpy()
    np.testing.assert_allclose(y, ops.layernorm(x, np.ones(768, np.float32),
                                                np.zeros(768, np.float32), 1e-5), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(y.mean(-1), 0, atol=1e-5)
    np.testing.assert_allclose(y.std(-1), 1, atol=1e-4)


@pytest.mark.parametrize("shape", [(4096, 3072), (3, 5), (1000,), (128, 768), (17, 24)])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("mode", ["tanh", "none"])
@pytest.mark.parametrize("with_bias", [False, True])
def test_gelu(dev, shape, dtype, mode, with_bias):
    from zenith_amd import zenith_cuda as zc

    x = synthetic.normal(shape, tag=5) * 3
    bias = synthetic.normal((shape[-1],), tag=6) if with_bias else None
    tdt = torch.float32 if dtype == "f32" else torch.float16
    if dtype == "f16":
        x = synthetic.round_f16(x)
        bias = None if bias is None else synthetic.round_f16(bias)
    tb = None if bias is None else _t(bias, dev, tdt)
    y = zc.bias_gelu(_t(x, dev, tdt), tb, approximate=mode).float().cpu().numpy()
    ref = ops.bias_gelu(x, bias, "tanh" if mode == "tanh" else "erf")
    if dtype == "f32":
        np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-6)
    else:
        ok, worst = fp16_tol(y, ref)
        assert ok, worst


def test_gelu_reference_kats(dev):
    """GELU(1) ~ 0.841, GELU(0) = 0, GELU(-1) ~ -0.159 (+-0.01), the reference's
    known answers (tests/test_cuda_cublas_bindings.py:36-57)."""
    from zenith_amd import zenith_cuda as zc

    y = zc.gelu(torch.tensor([1.0, 0.0, -1.0], device=dev)).cpu().numpy()
    assert abs(y[0] - 0.841) < 0.01 and y[1] == 0.0 and abs(y[2] + 0.159) < 0.01


@pytest.mark.parametrize("n", [1, 7, 4096 * 768 + 5])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_relu(dev, n, dtype):
    from zenith_amd import zenith_cuda as zc

    x = synthetic.normal((n,), tag=7)
    y = zc.relu(_t(x, dev, dtype)).float().cpu().numpy()
    np.testing.assert_array_equal(y, ops.relu(x.astype(np.float16 if dtype == torch.float16 else np.float32)).astype(np.float32))


@pytest.mark.parametrize("op", ["sigmoid", "tanh"])
@pytest.mark.parametrize("n", [1, 9, 4096 * 768 + 3])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("offset", [0, 1])
def test_sigmoid_tanh(dev, op, n, dtype, offset):
    """zk_sigmoid / zk_tanh through the C ABI: the vector body, the scalar
    tail, a misaligned start (offset 1 takes the scalar kernel), saturation
    at +-inf and large |x|, NaN propagation. fp32: a few ulp of the float32
    oracle; fp16: the fp16 bar on fp16-rounded inputs."""
    from zenith_amd import _lib as L

    x = synthetic.normal((n + offset,), tag=17) * 4
    x[offset: offset + 6] = np.array([0.0, -np.inf, np.inf, 100.0, -100.0, np.nan],
                                     np.float32)[: min(n, 6)]
    tdt = torch.float32 if dtype == "f32" else torch.float16
    if dtype == "f16":
        x = synthetic.round_f16(x)
    xt = _t(x, dev, tdt)[offset:]
    y = torch.empty_like(xt)
    L.call("zk_" + op, xt.data_ptr(), y.data_ptr(), n,
           L.ZK_F32 if dtype == "f32" else L.ZK_F16, torch.cuda.current_stream().cuda_stream)
    ref = getattr(ops, op)(x[offset:])
    y = y.float().cpu().numpy()
    assert np.array_equal(np.isnan(y), np.isnan(ref))
    ok = ~np.isnan(ref)
    if dtype == "f32":
        np.testing.assert_allclose(y[ok], ref[ok], rtol=2e-6, atol=1e-7)
    else:
        good, worst = fp16_tol(y[ok], ref[ok])
        assert good, worst
    if n >= 6 and offset == 0:
        sat = y[1:5]
        expect = [0.0, 1.0, 1.0, 0.0] if op == "sigmoid" else [-1.0, 1.0, 1.0, -1.0]
        assert sat.tolist() == expect and y[0] == (0.5 if op == "sigmoid" else 0.0)


@pytest.mark.parametrize("n", [1, 9, 4096 * 768, 4096 * 3072 + 3])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_quantize_bit_exact(dev, n, dtype):
    from zenith_amd import zenith_cuda as zc

    x = synthetic.normal((n,), tag=8) * 2
    if dtype == "f16":
        x = synthetic.round_f16(x)
    # ties: exact multiples of scale/2 must round half to even
    s = np.float32(0.0625)
    x[: min(n, 6)] = np.array([0.03125, 0.09375, -0.03125, -0.09375, 100.0, -100.0], np.float32)[: min(n, 6)]
    tdt = torch.float32 if dtype == "f32" else torch.float16
    q = zc.quantize_int8(_t(x, dev, tdt), float(s)).cpu().numpy()
    np.testing.assert_array_equal(q, ops.quantize_int8(x, s))
    s2 = ops.absmax_scale(np.abs(x).max())
    q2 = zc.quantize_int8(_t(x, dev, tdt), float(s2)).cpu().numpy()
    np.testing.assert_array_equal(q2, ops.quantize_int8(x, s2))

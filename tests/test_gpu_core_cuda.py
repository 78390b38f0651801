"""GPU parity: the GpuTensor API (`_zenith_core.cuda` mirror, python/src/
bindings.cpp:1367-2009) over the HIP kernels, and the reference's hybrid BERT
encoder written against it (benchmarks/bert_hybrid.py:96-168), vs the CPU
oracle. fp32 operations: rtol 1e-5 (matmul / linear / attention 1e-4);
fp16 variants: the fp16 bar on fp16-rounded inputs; layout and add: exact."""

import numpy as np
import pytest
import torch

from oracle import bert as obert
from oracle import ops
from tests.conftest import fp16_tol
from zenith_amd import synthetic

pytestmark = pytest.mark.gpu


def _c():
    from zenith_amd import core_cuda

    return core_cuda


def test_tensor_roundtrip(dev):
    cuda = _c()
    a = synthetic.normal((3, 5, 7), tag=1)
    t = cuda.to_gpu(a)
    assert t.is_valid() and t.shape == (3, 5, 7) and t.ndim() == 3 and t.dim(2) == 7
    assert t.numel() == 105 and t.size_bytes() == 420
    assert repr(t) == "GpuTensor(shape=[3, 5, 7], device=cuda)"
    np.testing.assert_array_equal(t.to_numpy(), a)
    assert cuda.empty((4, 2)).shape == (4, 2)
    with pytest.raises(RuntimeError):
        t.dim(3)


def test_elementwise_and_norm(dev):
    cuda = _c()
    x = synthetic.normal((64, 768), tag=2) * 2
    r = synthetic.normal((64, 768), tag=3)
    g = 1 + synthetic.normal((768,), tag=4, std=0.1)
    b = synthetic.normal((768,), tag=5, std=0.1)
    bias = synthetic.normal((768,), tag=6)
    X, R, G, B_ = (cuda.to_gpu(a) for a in (x, r, g, b))
    np.testing.assert_allclose(cuda.gelu_gpu(X).to_numpy(), ops.gelu_tanh(x), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(cuda.layernorm_gpu(X, G, B_).to_numpy(),
                               ops.layernorm(x, g, b, 1e-5), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(cuda.fused_add_layernorm_gpu(X, R, G, B_, 1e-12).to_numpy(),
                               ops.add_layernorm(x, r, g, b, 1e-12), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(cuda.fused_bias_gelu_gpu(X, cuda.to_gpu(bias)).to_numpy(),
                               ops.bias_gelu(x, bias, "tanh"), rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(cuda.add_2d_gpu(X, R).to_numpy(), x + r)


@pytest.mark.parametrize("rows,cols", [(64, 128), (7, 1000), (3, 5)])
def test_softmax(dev, rows, cols):
    cuda = _c()
    x = synthetic.normal((rows, cols), tag=7) * 10
    x[0, :] += 1000.0  # large logits: the max shift must keep it finite
    y = cuda.softmax_gpu(cuda.to_gpu(x)).to_numpy()
    np.testing.assert_allclose(y, ops.softmax(x), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(y.sum(-1), 1.0, rtol=1e-5)


def test_matmul_linear(dev):
    cuda = _c()
    a = synthetic.normal((100, 70), tag=8)
    bm = synthetic.normal((70, 37), tag=9)
    w = synthetic.normal((37, 70), tag=10)
    bias = synthetic.normal((37,), tag=11)
    A = cuda.to_gpu(a)
    np.testing.assert_allclose(cuda.matmul_gpu(A, cuda.to_gpu(bm)).to_numpy(), ops.matmul_f64(a, bm),
                               rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(cuda.linear_gpu(A, cuda.to_gpu(w), cuda.to_gpu(bias)).to_numpy(),
                               ops.matmul_f64(a, w.T) + bias, rtol=1e-4, atol=1e-4)
    # an invalid (or wrong-sized) bias is skipped, as in the reference
    np.testing.assert_allclose(cuda.linear_gpu(A, cuda.to_gpu(w), cuda.GpuTensor()).to_numpy(),
                               ops.matmul_f64(a, w.T), rtol=1e-4, atol=1e-4)
    with pytest.raises(RuntimeError):
        cuda.matmul_gpu(A, A)


@pytest.mark.parametrize("M,K,N", [(128, 256, 384), (1, 768, 3072), (300, 64, 200), (33, 12, 5)])
def test_matmul_paths(dev, M, K, N):
    """matmul_gpu / NumPy matmul: products with K % 4 == 0 and at least 2^18
    multiply-adds transpose B and run on the fp32 MFMA GEMM, the rest on the
    SIMT kernel; both against the float64-accumulated product."""
    cuda = _c()
    a = synthetic.normal((M, K), tag=30)
    b = synthetic.normal((K, N), tag=31)
    ref = ops.matmul_f64(a, b)
    np.testing.assert_allclose(cuda.matmul_gpu(cuda.to_gpu(a), cuda.to_gpu(b)).to_numpy(), ref,
                               rtol=1e-4, atol=1e-4)
    y = cuda.matmul(a, b)
    assert isinstance(y, np.ndarray) and y.dtype == np.float32 and y.shape == (M, N)
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-4)
    with pytest.raises(RuntimeError):
        cuda.matmul(a, a.T[:-1])


def test_onnx_branch_functions(dev):
    """What the ONNX operators' GPU branches call, in their order
    (activation_ops.py:52-181: upload with to_gpu, the *_gpu function, the
    module-level to_numpy; math_ops.py:83-190: NumPy matmul and 4D add), vs
    the operators' own NumPy formulas (the oracle)."""
    cuda = _c()
    assert cuda.is_available()
    x = synthetic.normal((2, 3, 5, 7), tag=32) * 3
    X = cuda.to_gpu(x)
    for name, ref, rtol in (("relu_gpu", ops.relu(x), 0), ("sigmoid_gpu", ops.sigmoid(x), 2e-6),
                            ("tanh_gpu", ops.tanh(x), 2e-6), ("gelu_gpu", ops.gelu_tanh(x), 1e-5)):
        y = cuda.to_numpy(getattr(cuda, name)(X))
        assert y.shape == x.shape and y.dtype == np.float32, name
        np.testing.assert_allclose(y, ref, rtol=rtol, atol=1e-6, err_msg=name)
    x2 = x.reshape(6, 35)
    np.testing.assert_allclose(cuda.to_numpy(cuda.softmax_gpu(cuda.to_gpu(x2))), ops.softmax(x2),
                               rtol=1e-5, atol=1e-7)
    with pytest.raises(RuntimeError):  # 2D only, as in the reference
        cuda.softmax_gpu(X)
    z = synthetic.normal(x.shape, tag=33)
    np.testing.assert_array_equal(cuda.add(x, z), x + z)
    np.testing.assert_array_equal(cuda.add_gpu(X, cuda.to_gpu(z)).to_numpy(), x + z)
    with pytest.raises(RuntimeError):
        cuda.add(x, z[:1])


def test_numpy_interface(dev):
    """NumPy-array functions (bindings.cpp:2010-2131 and the cuDNN-backed
    relu / add) vs the oracle."""
    cuda = _c()
    x = synthetic.normal((17, 768), tag=34) * 2
    g = 1 + synthetic.normal((768,), tag=35, std=0.1)
    b = synthetic.normal((768,), tag=36, std=0.1)
    np.testing.assert_array_equal(cuda.relu(x), ops.relu(x))
    np.testing.assert_allclose(cuda.gelu(x), ops.gelu_tanh(x), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(cuda.layernorm(x, g, b), ops.layernorm(x, g, b, 1e-5),
                               rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(cuda.layernorm(x, g, b, 1e-12), ops.layernorm(x, g, b, 1e-12),
                               rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(cuda.softmax(x), ops.softmax(x), rtol=1e-5, atol=1e-7)
    for fn, args in ((cuda.gelu, (x[0],)), (cuda.softmax, (x[0],)), (cuda.layernorm, (x[0], g, b))):
        with pytest.raises(RuntimeError):
            fn(*args)
    st = cuda.memory_stats()
    assert st["total_allocated"] > 0 and st["allocations"] > 0


def test_layout_ops(dev):
    cuda = _c()
    B, S, H, D = 2, 5, 3, 8
    x = synthetic.normal((B * S, H * D), tag=12)
    t4 = cuda.transpose_for_attention(cuda.to_gpu(x), B, S, H, D)
    assert t4.shape == (B, H, S, D)
    np.testing.assert_array_equal(t4.to_numpy(), x.reshape(B, S, H, D).transpose(0, 2, 1, 3))
    back = cuda.transpose_from_attention(t4, B, H, S, D)
    np.testing.assert_array_equal(back.to_numpy(), x.reshape(B, S, H, D))
    flat = cuda.reshape_4d_to_2d(back, B, S, H * D)
    assert flat.shape == (B * S, H * D)
    np.testing.assert_array_equal(flat.to_numpy(), x)
    # odd last dimension takes the scalar path
    y = synthetic.normal((2, 3, 4, 5), tag=13)
    np.testing.assert_array_equal(
        cuda.transpose_for_attention(cuda.to_gpu(y), 2, 3, 4, 5).to_numpy(), y.transpose(0, 2, 1, 3))


def test_attention_fp32_and_fp16(dev):
    cuda = _c()
    B, H, S, D = 2, 4, 128, 64
    q, k, v = (synthetic.normal((B, H, S, D), tag=20 + i) for i in range(3))
    Q, K, V = (cuda.to_gpu(a) for a in (q, k, v))
    ref = ops.attention(q, k, v)
    for fn in (cuda.flash_attention_gpu, cuda.cublas_attention_gpu):
        np.testing.assert_allclose(fn(Q, K, V).to_numpy(), ref, rtol=1e-4, atol=1e-5)
    ref16 = ops.attention(*(synthetic.round_f16(a) for a in (q, k, v)))
    for fn in (cuda.attention_fp16_gpu, cuda.attention_full_fp16_gpu):
        ok, worst = fp16_tol(fn(Q, K, V).to_numpy(), ref16)
        assert ok, worst


def test_fp16_variants(dev):
    cuda = _c()
    r16 = synthetic.round_f16
    x = synthetic.normal((128, 768), tag=30)
    w = synthetic.normal((256, 768), tag=31, std=0.03)
    bias = synthetic.normal((256,), tag=32)
    g = 1 + synthetic.normal((768,), tag=33, std=0.1)
    b = synthetic.normal((768,), tag=34, std=0.1)
    y = cuda.linear_fp16_gpu(cuda.to_gpu(x), cuda.to_gpu(w), cuda.to_gpu(bias)).to_numpy()
    ok, worst = fp16_tol(y, ops.matmul_f64(r16(x), r16(w).T) + r16(bias))
    assert ok, worst
    ok, worst = fp16_tol(cuda.gelu_fp16_gpu(cuda.to_gpu(x)).to_numpy(), ops.gelu_tanh(r16(x)))
    assert ok, worst
    ok, worst = fp16_tol(cuda.layernorm_fp16_gpu(cuda.to_gpu(x), cuda.to_gpu(g), cuda.to_gpu(b)).to_numpy(),
                         ops.layernorm(r16(x), r16(g), r16(b), 1e-5))
    assert ok, worst
    x2 = synthetic.normal((128, 768), tag=35)
    s = cuda.add_fp16_gpu(cuda.to_gpu(x), cuda.to_gpu(x2)).to_numpy()
    np.testing.assert_array_equal(s, (x.astype(np.float16) + x2.astype(np.float16)).astype(np.float32))


def test_convert_round_to_nearest_even(dev):
    """zk_convert fp32 -> fp16 equals numpy's round-to-nearest-even cast,
    including ties, subnormals, overflow to inf; fp16 -> fp32 is exact."""
    from zenith_amd import _lib as L

    rng = np.random.default_rng(3)
    x = np.concatenate([rng.normal(0, 100, 4093).astype(np.float32),
                        np.float32([65504, 65520, 70000, 6e-8, 3e-8, -0.0, 1 + 2**-11, 1 + 3 * 2**-11])])
    xt = torch.from_numpy(x).to(dev)
    h = torch.empty(x.size, dtype=torch.float16, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    L.call("zk_convert", xt.data_ptr(), h.data_ptr(), x.size, L.ZK_F32, L.ZK_F16, st)
    np.testing.assert_array_equal(h.cpu().numpy().view(np.uint16), x.astype(np.float16).view(np.uint16))
    back = torch.empty_like(xt)
    L.call("zk_convert", h.data_ptr(), back.data_ptr(), x.size, L.ZK_F16, L.ZK_F32, st)
    np.testing.assert_array_equal(back.cpu().numpy(), x.astype(np.float16).astype(np.float32))


def test_hybrid_encoder_vs_oracle(dev):
    """Two hybrid layers (fp32 linears, fp16 attention, tanh GELU, eps 1e-5)
    vs the fp32 oracle layer with the same settings."""
    from zenith_amd.bert_hybrid import BertEncoderHybrid

    B, S = 2, 128
    w = synthetic.bert_weights(2, seed=5)
    x = synthetic.hidden_states(B, S, seed=5)
    enc = BertEncoderHybrid(num_layers=2).load_weights(w)
    from zenith_amd import core_cuda as cuda

    y = enc.forward(cuda.to_gpu(x.reshape(B * S, 768)), B, S).to_numpy().reshape(B, S, 768)
    ref = obert.bert_encoder(x, w, eps=1e-5, gelu="tanh")
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert rel < 2e-2 and np.all(np.abs(y - ref) <= 2e-2 + 2e-2 * np.abs(ref)), rel


def test_hybrid_encoder_vs_transformers(dev):
    """The reference's own accuracy check (bert_hybrid.py:210-231): a
    12-layer transformers BertModel encoder (hidden_act gelu_new, random
    init, seed 42) against the hybrid encoder loaded from it, b=1 s=128;
    the reference reports max_diff 7.1e-4 on a T4 (BENCHMARK_REPORT.md:60)."""
    transformers = pytest.importorskip("transformers")
    from zenith_amd import core_cuda as cuda
    from zenith_amd.bert_hybrid import BertEncoderHybrid

    torch.manual_seed(42)
    cfg = transformers.BertConfig(hidden_size=768, num_attention_heads=12, intermediate_size=3072,
                                  num_hidden_layers=12, hidden_act="gelu_new")
    cfg._attn_implementation = "eager"
    model = transformers.BertModel(cfg).eval()
    x = np.random.default_rng(42).standard_normal((1, 128, 768)).astype(np.float32)
    with torch.no_grad():
        ref = model.encoder(torch.from_numpy(x))[0].numpy()
    enc = BertEncoderHybrid(12).load_from_pytorch(model.encoder)
    y = enc.forward(cuda.to_gpu(x.reshape(128, 768)), 1, 128).to_numpy().reshape(1, 128, 768)
    # HF LayerNorm eps is 1e-12, the hybrid's fused Add+LN call uses 1e-5
    assert np.max(np.abs(y - ref)) < 5e-3, np.max(np.abs(y - ref))

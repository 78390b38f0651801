"""CPU checks of the GpuTensor API surface (python/src/bindings.cpp:694-781):
invalid tensors and precondition errors raise RuntimeError before any GPU
work, as the reference's bindings do."""

import pytest

from zenith_amd import core_cuda as cuda


def test_invalid_gpu_tensor():
    t = cuda.GpuTensor()
    assert not t.is_valid()
    assert t.numel() == 0 and t.size_bytes() == 0 and t.ndim() == 0 and t.shape == ()
    assert repr(t) == "GpuTensor(invalid)"
    with pytest.raises(RuntimeError):
        t.dim(0)
    with pytest.raises(RuntimeError):
        t.to_numpy()


@pytest.mark.parametrize("fn,args", [
    (cuda.gelu_gpu, 1), (cuda.layernorm_gpu, 3), (cuda.matmul_gpu, 2), (cuda.linear_gpu, 3),
    (cuda.softmax_gpu, 1), (cuda.flash_attention_gpu, 3), (cuda.cublas_attention_gpu, 3),
    (cuda.add_2d_gpu, 2), (cuda.fused_add_layernorm_gpu, 4), (cuda.fused_bias_gelu_gpu, 2),
    (cuda.attention_fp16_gpu, 3), (cuda.attention_full_fp16_gpu, 3), (cuda.linear_fp16_gpu, 3),
    (cuda.gelu_fp16_gpu, 1), (cuda.layernorm_fp16_gpu, 3), (cuda.add_fp16_gpu, 2),
    (cuda.relu_gpu, 1), (cuda.sigmoid_gpu, 1), (cuda.tanh_gpu, 1), (cuda.add_gpu, 2),
])
def test_invalid_inputs_raise(fn, args):
    with pytest.raises(RuntimeError):
        fn(*[cuda.GpuTensor() for _ in range(args)])


def test_layout_ops_reject_invalid():
    with pytest.raises(RuntimeError):
        cuda.transpose_for_attention(cuda.GpuTensor(), 1, 2, 3, 4)
    with pytest.raises(RuntimeError):
        cuda.transpose_from_attention(cuda.GpuTensor(), 1, 2, 3, 4)
    with pytest.raises(RuntimeError):
        cuda.reshape_4d_to_2d(cuda.GpuTensor(), 1, 2, 3)


def test_gpu_tensor_rejects_cpu_data():
    import torch

    with pytest.raises(RuntimeError):
        cuda.GpuTensor(torch.zeros(3))


def test_onnx_branch_surface():
    """Every function the ONNX operators' GPU branches and ExecutionContext
    call on ``_zenith_core.cuda`` (activation_ops.py:52-181,
    math_ops.py:83-190, context.py:56-182) exists with the reference's name."""
    for name in ("is_available", "to_gpu", "to_numpy", "relu_gpu", "sigmoid_gpu", "tanh_gpu",
                 "softmax_gpu", "gelu_gpu", "matmul", "add"):
        assert callable(getattr(cuda, name)), name
    with pytest.raises(RuntimeError):
        cuda.to_numpy(cuda.GpuTensor())
    with pytest.raises(RuntimeError):
        cuda.to_numpy([1.0])


def test_no_gpu_reports_unavailable():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    assert cuda.is_available() is False
    assert set(cuda.memory_stats()) == {"allocations", "cache_hits", "cache_returns",
                                        "total_allocated"}
    for fn, args in ((cuda.matmul, ([[1.0]], [[1.0]])), (cuda.add, ([1.0], [1.0])),
                     (cuda.relu, ([1.0],)), (cuda.softmax, ([[1.0]],))):
        with pytest.raises(RuntimeError):
            fn(*args)

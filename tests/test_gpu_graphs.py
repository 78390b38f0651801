"""GPU: the HIP-graph manager with the zenith_amd kernels. Every replay is
compared bit for bit with the eager result, with eager work between
replays; the hybrid encoder (GpuTensor API) is replayed through
make_graphed_callable."""

import numpy as np
import pytest
import torch

from zenith_amd import synthetic

pytestmark = pytest.mark.gpu


def test_capture_replay_lru_and_stats(dev):
    from zenith_amd import graphs
    from zenith_amd import zenith_cuda as zc

    m = graphs.CudaGraphManager(max_cached_graphs=2)
    x = torch.randn(256, 768, device=dev, dtype=torch.float16)
    g = torch.randn(768, device=dev, dtype=torch.float16)
    b = torch.randn(768, device=dev, dtype=torch.float16)
    eager = zc.gelu(zc.layernorm(x, g, b, 1e-5)).clone()
    with m.capture("ln_gelu"):
        out = zc.gelu(zc.layernorm(x, g, b, 1e-5))
    for _ in range(3):
        assert m.replay("ln_gelu")
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        zc.relu(x)  # eager work between replays
    st = m.get_statistics("ln_gelu")
    assert st.launch_count == 3 and st.average_time_ms > 0
    with m.capture("a"):
        zc.relu(x)
    with m.capture("b"):
        zc.relu(x)
    assert m.cache_size == 2 and m.get_statistics("ln_gelu") is None  # LRU evicted
    assert m.invalidate("a") and m.cache_size == 1
    assert m.clear() == 1


def test_graph_cached_decorator(dev):
    from zenith_amd import graphs
    from zenith_amd import zenith_cuda as zc

    m = graphs.CudaGraphManager(warmup_iterations=2)
    x = torch.randn(4096, device=dev, dtype=torch.float16)

    @m.graph_cached("relu_gelu")
    def f(t):
        return zc.gelu(zc.relu(t))

    ref = zc.gelu(zc.relu(x)).clone()
    outs = [f(x).clone() for _ in range(5)]  # 2 eager, 1 capture + replay, 2 replays
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o, ref)
    x.mul_(-1)  # same memory, new values: the replay sees them
    ref2 = zc.gelu(zc.relu(x)).clone()
    assert torch.equal(f(x), ref2)
    assert m.get_statistics("relu_gelu").launch_count == 4


def test_hybrid_encoder_graphed(dev):
    from zenith_amd import core_cuda as cuda
    from zenith_amd import graphs
    from zenith_amd.bert_hybrid import BertEncoderHybrid

    B, S = 1, 128
    enc = BertEncoderHybrid(num_layers=2).load_weights(synthetic.bert_weights(2, seed=3))
    x1 = cuda.to_gpu(synthetic.hidden_states(B, S, seed=3).reshape(B * S, 768))
    x2 = cuda.to_gpu(synthetic.hidden_states(B, S, seed=4).reshape(B * S, 768))
    e1 = enc.forward(x1, B, S).to_numpy()
    e2 = enc.forward(x2, B, S).to_numpy()
    m = graphs.CudaGraphManager()
    fwd = m.make_graphed_callable(enc.forward, (x1, B, S), key="hybrid")
    for xin, ref in ((x2, e2), (x1, e1), (x2, e2)):
        out = fwd(xin, B, S)
        np.testing.assert_array_equal(out.to_numpy(), ref)


def test_cached_graph_model(dev):
    from zenith_amd import graphs
    from zenith_amd import zenith_cuda as zc

    model = graphs.CachedGraphModel(lambda t: zc.relu(zc.gelu(t)), warmup_iterations=1)
    a = torch.randn(1000, device=dev)
    b = torch.randn(1000, device=dev)
    ra, rb = zc.relu(zc.gelu(a)).clone(), zc.relu(zc.gelu(b)).clone()
    for t, r in ((a, ra), (b, rb), (a, ra), (b, rb)):
        assert torch.equal(model(t), r)
    c = torch.randn(10, device=dev)  # another shape: its own graph
    assert torch.equal(model(c), zc.relu(zc.gelu(c)))
    assert len(model.statistics) >= 1

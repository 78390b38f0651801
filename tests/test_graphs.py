"""CPU checks of the graph manager (zenith/runtime/cuda_graphs.py:65-846
mirror): without a GPU graphs are disabled and every wrapper runs its
function eagerly, as the reference's does."""

import warnings

from zenith_amd import graphs


def _mgr(**kw):
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", RuntimeWarning)
        return graphs.CudaGraphManager(**kw)


def test_disabled_without_gpu():
    m = _mgr()
    assert not m.graphs_enabled and m.cache_size == 0 and m.total_launches == 0
    assert m.replay("nothing") is False
    assert m.get_statistics("nothing") is None
    assert m.invalidate("nothing") is False and m.clear() == 0
    with m.capture("k") as ctx:  # no capture happens
        assert ctx.stream is None
    assert m.cache_size == 0


def test_wrappers_run_eagerly():
    m = _mgr(warmup_iterations=1)
    calls = []

    @m.graph_cached("f")
    def f(x):
        calls.append(x)
        return x * 2

    assert [f(i) for i in range(3)] == [0, 2, 4] and calls == [0, 1, 2]
    g = m.make_graphed_callable(lambda a: a + 1, (1,))
    assert g(5) == 6
    model = graphs.CachedGraphModel(lambda a: a - 1, warmup_iterations=1)
    assert model(3) == 2 and model(4) == 3


def test_enums_and_stats():
    s = graphs.GraphStatistics(launch_count=4, total_time_ms=2.0)
    s.update_average()
    assert s.average_time_ms == 0.5
    assert graphs.GraphStatus.INSTANTIATED.value == "instantiated"
    assert graphs.GraphCaptureMode.RELAXED.value == "relaxed"

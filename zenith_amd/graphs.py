"""HIP-graph capture / replay manager.

Mirrors the reference's CUDA-graph runtime (zenith/runtime/cuda_graphs.py:
65-846): GraphCaptureMode, GraphStatus, GraphStatistics, CachedGraph,
CudaGraphManager (capture / replay / invalidate / clear / statistics /
graph_cached / make_graphed_callable, LRU eviction), GraphCaptureContext,
CachedGraphModel and the module-level get_global_manager / capture / replay /
graph_cached. The graphs are torch.cuda.CUDAGraph objects, i.e. HIP graphs on
ROCm, and every zenith_amd kernel launches on torch's current stream, so a
capture records the HIP kernels directly.

Differences from the reference, by design:
  - capture runs on a side stream that first waits for the caller's stream
    (a graph cannot be captured on the legacy default stream); replays go
    to the caller's stream;
  - replay statistics record a pair of HIP events per replay and resolve
    them when statistics are read, instead of synchronising the host after
    every replay (cuda_graphs.py:283-297);
  - graphed callables also take GpuTensor arguments (zenith_amd.core_cuda),
    whose device memory is copied into the static inputs before a replay.
Captured work must not record hipMemsetAsync nodes (the zenith_amd kernels
record none); buffers that must start at zero are cleared by kernels.
"""

from __future__ import annotations

import functools
import hashlib
import threading
import time
import warnings
from dataclasses import dataclass, field
from enum import Enum
from typing import Any, Callable, Optional, TypeVar

F = TypeVar("F", bound=Callable[..., Any])


class GraphCaptureMode(Enum):
    GLOBAL = "global"
    THREAD_LOCAL = "thread_local"
    RELAXED = "relaxed"


class GraphStatus(Enum):
    NOT_CAPTURED = "not_captured"
    CAPTURING = "capturing"
    CAPTURED = "captured"
    INSTANTIATED = "instantiated"
    INVALID = "invalid"


@dataclass
class GraphStatistics:
    node_count: int = 0
    launch_count: int = 0
    total_time_ms: float = 0.0
    average_time_ms: float = 0.0
    capture_time_ms: float = 0.0

    def update_average(self) -> None:
        if self.launch_count > 0:
            self.average_time_ms = self.total_time_ms / self.launch_count


@dataclass
class CachedGraph:
    key: str
    status: GraphStatus = GraphStatus.NOT_CAPTURED
    statistics: GraphStatistics = field(default_factory=GraphStatistics)
    input_shapes: tuple = field(default_factory=tuple)
    graph_handle: Optional[Any] = None
    exec_handle: Optional[Any] = None
    static_inputs: Optional[list[Any]] = None
    static_outputs: Optional[Any] = None
    pending_events: list = field(default_factory=list)


def _torch():
    import torch

    return torch


class CudaGraphManager:
    """Keyed cache of captured HIP graphs with LRU eviction and statistics."""

    def __init__(self, max_cached_graphs: int = 100, warmup_iterations: int = 3,
                 enable_stats: bool = True):
        self._cache: dict[str, CachedGraph] = {}
        self._order: list[str] = []
        self._max_cached = max(1, int(max_cached_graphs))
        self._warmup_iterations = warmup_iterations
        self._enable_stats = enable_stats
        self._lock = threading.RLock()
        try:
            self._cuda_available = bool(_torch().cuda.is_available())
        except ImportError:  # pragma: no cover - torch is a dependency
            self._cuda_available = False
        if not self._cuda_available:
            warnings.warn("No GPU: HIP graphs are disabled and functions run eagerly.",
                          RuntimeWarning, stacklevel=2)

    # -- state -------------------------------------------------------------
    @property
    def cuda_available(self) -> bool:
        return self._cuda_available

    @property
    def graphs_enabled(self) -> bool:
        return self._cuda_available

    @property
    def cache_size(self) -> int:
        with self._lock:
            return len(self._cache)

    @property
    def total_launches(self) -> int:
        with self._lock:
            return sum(self._stats(c).launch_count for c in self._cache.values())

    def _touch(self, key: str) -> None:
        if key in self._order:
            self._order.remove(key)
        self._order.append(key)

    def _evict_for_new(self) -> None:
        while len(self._cache) >= self._max_cached and self._order:
            self._cache.pop(self._order.pop(0), None)

    # -- capture -----------------------------------------------------------
    def capture(self, key: str, stream: Optional[Any] = None,
                mode: GraphCaptureMode = GraphCaptureMode.GLOBAL,
                pool: Optional[Any] = None) -> "GraphCaptureContext":
        """Context manager: the work inside is captured under `key`."""
        return GraphCaptureContext(self, key, stream, mode, pool)

    def _begin(self, key: str, stream, mode: GraphCaptureMode, pool):
        torch = _torch()
        with self._lock:
            self._evict_for_new()
            entry = CachedGraph(key=key, status=GraphStatus.CAPTURING)
            self._cache[key] = entry
            self._touch(key)
        graph = torch.cuda.CUDAGraph()
        entry.graph_handle = graph
        caller = stream if stream is not None else torch.cuda.current_stream()
        side = torch.cuda.Stream(device=caller.device)
        side.wait_stream(caller)
        t0 = time.perf_counter()
        ctx = torch.cuda.graph(graph, pool=pool, stream=side,
                               capture_error_mode=mode.value)
        ctx.__enter__()
        return entry, ctx, caller, side, t0

    def _end(self, state, failed: bool) -> None:
        entry, ctx, caller, side, t0 = state
        if failed:
            ctx.__exit__(RuntimeError, RuntimeError("capture failed"), None)
        else:
            ctx.__exit__(None, None, None)
        caller.wait_stream(side)
        if failed:
            self.invalidate(entry.key)
            return
        with self._lock:
            entry.exec_handle = entry.graph_handle
            entry.status = GraphStatus.INSTANTIATED
            entry.statistics.node_count = 1
            entry.statistics.capture_time_ms = (time.perf_counter() - t0) * 1e3  # host time

    # -- replay ------------------------------------------------------------
    def replay(self, key: str, stream: Optional[Any] = None) -> bool:
        """Launch the graph cached under `key` on `stream` (default: the
        current stream). False when no such graph exists; ValueError when it
        is not instantiated."""
        torch = _torch()
        with self._lock:
            entry = self._cache.get(key)
            if entry is None:
                return False
            if entry.status != GraphStatus.INSTANTIATED:
                raise ValueError(f"Graph '{key}' is not instantiated. Status: {entry.status}")
            if not self.graphs_enabled:
                return False
            self._touch(key)
        s = stream if stream is not None else torch.cuda.current_stream()
        if self._enable_stats:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            with torch.cuda.stream(s):
                entry.exec_handle.replay()
            e1.record(s)
            with self._lock:
                entry.statistics.launch_count += 1
                entry.pending_events.append((e0, e1))
                self._fold_done(entry)
        else:
            with torch.cuda.stream(s):
                entry.exec_handle.replay()
        return True

    # -- bookkeeping ---------------------------------------------------------
    def invalidate(self, key: str) -> bool:
        with self._lock:
            entry = self._cache.pop(key, None)
            if key in self._order:
                self._order.remove(key)
            if entry is None:
                return False
            entry.status = GraphStatus.INVALID
            entry.graph_handle = entry.exec_handle = None
            entry.static_inputs = entry.static_outputs = None
            return True

    def clear(self) -> int:
        with self._lock:
            n = len(self._cache)
            self._cache.clear()
            self._order.clear()
            return n

    @staticmethod
    def _fold_done(entry: CachedGraph) -> None:
        """Fold the replays that have finished into the totals, without
        waiting, so the event list stays short when nobody reads statistics."""
        pend = entry.pending_events
        while pend and pend[0][1].query():
            e0, e1 = pend.pop(0)
            entry.statistics.total_time_ms += e0.elapsed_time(e1)
        entry.statistics.update_average()

    def _stats(self, entry: CachedGraph) -> GraphStatistics:
        """Resolve the replay events recorded so far (waits for them)."""
        if entry.pending_events:
            for e0, e1 in entry.pending_events:
                e1.synchronize()
                entry.statistics.total_time_ms += e0.elapsed_time(e1)
            entry.pending_events.clear()
            entry.statistics.update_average()
        return entry.statistics

    def get_statistics(self, key: str) -> Optional[GraphStatistics]:
        with self._lock:
            entry = self._cache.get(key)
            return None if entry is None else self._stats(entry)

    def get_all_statistics(self) -> dict[str, GraphStatistics]:
        with self._lock:
            return {k: self._stats(e) for k, e in self._cache.items()}

    # -- wrappers ----------------------------------------------------------
    def graph_cached(self, key: Optional[str] = None, warmup: Optional[int] = None
                     ) -> Callable[[F], F]:
        """Decorator: `warmup` eager calls, then one captured call, then
        replays that return the captured call's (static) outputs. The
        function's inputs must live in the same memory on every call."""

        def decorator(func: F) -> F:
            gkey = key or func.__name__
            n_warm = self._warmup_iterations if warmup is None else warmup
            state = {"calls": 0, "out": None, "captured": False}

            @functools.wraps(func)
            def wrapper(*args: Any, **kwargs: Any) -> Any:
                if not self.graphs_enabled:
                    return func(*args, **kwargs)
                state["calls"] += 1
                if state["calls"] <= n_warm:
                    return func(*args, **kwargs)
                if not state["captured"] or gkey not in self._cache:
                    with self.capture(gkey):
                        state["out"] = func(*args, **kwargs)
                    state["captured"] = True
                    self.replay(gkey)  # capture records, it does not run
                    return state["out"]
                self.replay(gkey)
                return state["out"]

            return wrapper  # type: ignore[return-value]

        return decorator

    def make_graphed_callable(self, func: Callable[..., Any], sample_args: tuple,
                              sample_kwargs: Optional[dict] = None, key: Optional[str] = None,
                              num_warmup: int = 3) -> Callable[..., Any]:
        """Capture func on static copies of the sample arguments; the returned
        callable copies its tensor arguments (torch tensors or GpuTensors)
        into those buffers, replays, and returns the static outputs."""
        if not self.graphs_enabled:
            return func
        torch = _torch()
        sample_kwargs = sample_kwargs or {}
        gkey = key or f"graphed_{id(func)}"
        static_args = tuple(_static_copy(a) for a in sample_args)
        static_kwargs = {k: _static_copy(v) for k, v in sample_kwargs.items()}
        with torch.no_grad():
            for _ in range(num_warmup):
                func(*static_args, **static_kwargs)
            torch.cuda.synchronize()
            with self.capture(gkey):
                out = func(*static_args, **static_kwargs)
        with self._lock:
            self._cache[gkey].static_inputs = list(static_args)
            self._cache[gkey].static_outputs = out

        def graphed(*args: Any, **kwargs: Any) -> Any:
            for a, s in zip(args, static_args):
                _copy_into(s, a)
            for k, v in kwargs.items():
                if k in static_kwargs:
                    _copy_into(static_kwargs[k], v)
            self.replay(gkey)
            return out

        return graphed


def _tensor_of(x):
    from .core_cuda import GpuTensor

    if isinstance(x, GpuTensor):
        return x.tensor if x.is_valid() else None
    torch = _torch()
    return x if isinstance(x, torch.Tensor) else None


def _static_copy(x):
    from .core_cuda import GpuTensor

    if isinstance(x, GpuTensor) and x.is_valid():
        return GpuTensor(x.tensor.clone())
    t = _tensor_of(x)
    return t.clone() if t is not None else x


def _copy_into(static, value) -> None:
    dst, src = _tensor_of(static), _tensor_of(value)
    if dst is not None and src is not None and dst.data_ptr() != src.data_ptr():
        if dst.shape != src.shape:
            raise RuntimeError(f"graphed callable: input shape {tuple(src.shape)} differs from "
                               f"the captured {tuple(dst.shape)}")
        dst.copy_(src)


class GraphCaptureContext:
    """`with manager.capture(key):` -- the work inside is captured."""

    def __init__(self, manager: CudaGraphManager, key: str, stream: Optional[Any],
                 mode: GraphCaptureMode, pool: Optional[Any]):
        self._manager, self._key, self._stream = manager, key, stream
        self._mode, self._pool = mode, pool
        self._state = None

    def __enter__(self) -> "GraphCaptureContext":
        if self._manager.graphs_enabled:
            self._state = self._manager._begin(self._key, self._stream, self._mode, self._pool)
        return self

    def __exit__(self, exc_type, exc_val, exc_tb) -> bool:
        if self._state is not None:
            self._manager._end(self._state, failed=exc_type is not None)
        return False

    @property
    def stream(self) -> Optional[Any]:
        return None if self._state is None else self._state[3]


class CachedGraphModel:
    """Model wrapper: per input-shape key, `warmup_iterations` eager calls,
    one capture, then replays returning the static outputs. Inputs are
    copied into the captured call's inputs before each replay."""

    def __init__(self, model: Any, warmup_iterations: int = 3, cache_by_shape: bool = True):
        self._model = model
        self._manager = CudaGraphManager(warmup_iterations=warmup_iterations)
        self._by_shape = cache_by_shape
        self._warm: dict[str, int] = {}
        self._static: dict[str, tuple] = {}
        self._lock = threading.RLock()

    @staticmethod
    def _shape_key(args: tuple, kwargs: dict) -> str:
        parts = []
        for a in args:
            t = _tensor_of(a)
            parts.append(str(tuple(t.shape)) if t is not None else type(a).__name__)
        for k, v in sorted(kwargs.items()):
            t = _tensor_of(v)
            if t is not None:
                parts.append(f"{k}:{tuple(t.shape)}")
        return hashlib.sha256("_".join(parts).encode()).hexdigest()[:16]

    def __call__(self, *args: Any, **kwargs: Any) -> Any:
        if not self._manager.graphs_enabled:
            return self._model(*args, **kwargs)
        key = f"model_{self._shape_key(args, kwargs)}" if self._by_shape else "model_default"
        with self._lock:
            left = self._warm.setdefault(key, self._manager._warmup_iterations)
            if left > 0:
                self._warm[key] = left - 1
                return self._model(*args, **kwargs)
            if key not in self._static or key not in self._manager._cache:
                s_args = tuple(_static_copy(a) for a in args)
                s_kwargs = {k: _static_copy(v) for k, v in kwargs.items()}
                with self._manager.capture(key):
                    out = self._model(*s_args, **s_kwargs)
                self._static[key] = (s_args, s_kwargs, out)
            s_args, s_kwargs, out = self._static[key]
            for a, s in zip(args, s_args):
                _copy_into(s, a)
            for k, v in kwargs.items():
                if k in s_kwargs:
                    _copy_into(s_kwargs[k], v)
            self._manager.replay(key)
            return out

    def invalidate(self) -> None:
        with self._lock:
            self._manager.clear()
            self._static.clear()
            self._warm.clear()

    @property
    def statistics(self) -> dict[str, GraphStatistics]:
        return self._manager.get_all_statistics()


_global: Optional[CudaGraphManager] = None
_global_lock = threading.Lock()


def get_global_manager() -> CudaGraphManager:
    global _global
    with _global_lock:
        if _global is None:
            _global = CudaGraphManager()
        return _global


def capture(key: str, stream: Optional[Any] = None,
            mode: GraphCaptureMode = GraphCaptureMode.GLOBAL) -> GraphCaptureContext:
    return get_global_manager().capture(key, stream, mode)


def replay(key: str, stream: Optional[Any] = None) -> bool:
    return get_global_manager().replay(key, stream)


def graph_cached(key: Optional[str] = None, warmup: Optional[int] = None) -> Callable[[F], F]:
    return get_global_manager().graph_cached(key, warmup)


__all__ = [
    "GraphCaptureMode", "GraphStatus", "GraphStatistics", "CachedGraph", "CudaGraphManager",
    "GraphCaptureContext", "CachedGraphModel", "get_global_manager", "capture", "replay",
    "graph_cached",
]

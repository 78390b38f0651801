"""Graph hooks that route the reference's graph-level op types and torch.fx
patterns to the HIP kernels: FX patterns + optimizer, torch.compile
backend, kernel registry and node dispatcher (the reference's
zenith/optimization/fx_patterns.py, fx_optimizer.py, zenith/runtime/
kernel_registry.py, dispatcher.py and adapters/pytorch_adapter.py:606-744,
restricted to the encoder kernel path)."""

from .backend import create_compile_backend, register_backend  # noqa: F401
from .dispatcher import (  # noqa: F401
    ExecutionContext,
    KernelDispatcher,
    KernelExecutionError,
    Node,
    UnsupportedOperationError,
)
from .fx_optimizer import FXOptimizer, OptimizationStats, optimize_fx_graph  # noqa: F401
from .fx_patterns import FXPattern, get_all_patterns  # noqa: F401
from .kernel_registry import KernelRegistry, KernelSpec, Precision, get_registry, reset_registry  # noqa: F401

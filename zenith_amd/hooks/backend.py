"""torch.compile backend that applies the FX rewrites.

Mirrors `PyTorchAdapter.create_compile_backend` (zenith/adapters/
pytorch_adapter.py:606-744) and `register_backend`
(zenith/integrations/torch_dynamo.py:80-144) for the kernel path only:

  opt_level <= 1, or fewer than 10 graph nodes -> the graph runs unchanged
                                                  (pytorch_adapter.py:663-667)
  opt_level >= 2 -> FX rewrites (SDPA -> HIP flash attention, Linear+GELU ->
                    fused GEMM epilogue, Add+LayerNorm, LayerNorm, GELU)
  precision "fp16" -> the graph module is cast to half (pytorch_adapter.py:
                    692-693)

The reference ran its FX rewrites only at opt_level >= 3 while registering
the backend with opt_level 2 (torch_dynamo.py:36,84), so its default never
reached a kernel; here the rewrites start at the default level 2. The
reference's Triton / autocast phase has no counterpart (no other code
generators on this path).
"""

from __future__ import annotations

import logging
import warnings
from typing import Callable, Optional

import torch

from .fx_optimizer import FXOptimizer

logger = logging.getLogger("zenith_amd.hooks.backend")

DEFAULT_OPT_LEVEL = 2


def create_compile_backend(target: str = "cuda", precision: str = "fp32",
                           opt_level: Optional[int] = None, **kwargs) -> Callable:
    level = DEFAULT_OPT_LEVEL if opt_level is None else int(opt_level)

    def zenith_backend(gm: torch.fx.GraphModule, example_inputs: list):
        zenith_backend.compiled_graphs += 1
        nodes = len(list(gm.graph.nodes))
        if level <= 1 or nodes < 10:
            zenith_backend.last_graph = gm
            return gm.forward
        if level >= 2 and target.startswith("cuda"):
            opt = FXOptimizer(**kwargs)
            gm = opt.optimize(gm, example_inputs)
            zenith_backend.last_stats = opt.get_stats()
            logger.info("zenith_amd backend: %s", opt.get_stats())
        if precision == "fp16":
            gm = gm.half()
        zenith_backend.last_graph = gm
        return gm.forward

    # the statistics and the rewritten GraphModule of the last graph compiled,
    # and how many graphs dynamo has handed over
    zenith_backend.last_stats = None
    zenith_backend.last_graph = None
    zenith_backend.compiled_graphs = 0
    return zenith_backend


# backends this module registered, by name: replacing one of these is silent
_REGISTERED: dict[str, Callable] = {}


def register_backend(name: str = "zenith", replace: bool = True, **kwargs) -> Callable:
    """Register the backend with torch._dynamo under `name` and return it.

    The reference's `import zenith` already registers a backend called
    "zenith" (zenith/integrations/torch_dynamo.py:158-170), and dynamo
    refuses a second registration of a name. With replace=True (default) an
    existing registration of `name` is removed first, so
    torch.compile(backend="zenith") reaches these kernels; a registration
    this module did not make is replaced with a warning. With replace=False
    a taken name raises RuntimeError instead of being silently kept.
    Removing a registration uses dynamo's backend tables; a torch release
    without them raises RuntimeError rather than guessing."""
    from torch._dynamo.backends import registry as _r

    backend = create_compile_backend(**kwargs)
    fns = getattr(_r, "_COMPILER_FNS", None)
    taken = name in _r.list_backends(exclude_tags=()) or (fns is not None and name in fns)
    if taken:
        if not replace:
            raise RuntimeError(f"a torch.compile backend named {name!r} is already registered")
        if fns is None:
            raise RuntimeError(f"cannot replace the torch.compile backend {name!r}: this torch "
                               "release has no dynamo backend table to remove it from")
        current = fns.get(name)
        if current is None or current is not _REGISTERED.get(name):
            warnings.warn(f"replacing the torch.compile backend registered as {name!r} "
                          "with the zenith_amd HIP backend", RuntimeWarning, stacklevel=2)
        fns.pop(name, None)
        getattr(_r, "_BACKENDS", {}).pop(name, None)
    _r.register_backend(compiler_fn=backend, name=name)
    _REGISTERED[name] = backend
    return backend

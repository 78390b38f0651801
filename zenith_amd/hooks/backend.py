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
from typing import Callable, Optional

import torch

from .fx_optimizer import FXOptimizer

logger = logging.getLogger("zenith_amd.hooks.backend")

DEFAULT_OPT_LEVEL = 2


def create_compile_backend(target: str = "cuda", precision: str = "fp32",
                           opt_level: Optional[int] = None, **kwargs) -> Callable:
    level = DEFAULT_OPT_LEVEL if opt_level is None else int(opt_level)

    def zenith_backend(gm: torch.fx.GraphModule, example_inputs: list):
        nodes = len(list(gm.graph.nodes))
        if level <= 1 or nodes < 10:
            return gm.forward
        if level >= 2 and target.startswith("cuda"):
            opt = FXOptimizer(**kwargs)
            gm = opt.optimize(gm, example_inputs)
            zenith_backend.last_stats = opt.get_stats()
            logger.info("zenith_amd backend: %s", opt.get_stats())
        if precision == "fp16":
            gm = gm.half()
        return gm.forward

    zenith_backend.last_stats = None
    return zenith_backend


def register_backend(name: str = "zenith", replace: bool = True, **kwargs) -> Callable:
    """Register the backend with torch._dynamo under `name` and return it.

    The reference's `import zenith` already registers a backend called
    "zenith" (zenith/integrations/torch_dynamo.py:158-170), and dynamo
    refuses a second registration of a name. With replace=True (default) an
    existing registration of `name` is removed first, so
    torch.compile(backend="zenith") reaches these kernels; with replace=False
    a taken name raises RuntimeError instead of being silently kept."""
    from torch._dynamo.backends import registry as _r

    backend = create_compile_backend(**kwargs)
    taken = name in _r._COMPILER_FNS or name in _r.list_backends(exclude_tags=())
    if taken:
        if not replace:
            raise RuntimeError(f"a torch.compile backend named {name!r} is already registered")
        _r._COMPILER_FNS.pop(name, None)
        _r._BACKENDS.pop(name, None)
    _r.register_backend(compiler_fn=backend, name=name)
    return backend

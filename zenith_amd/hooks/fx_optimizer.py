"""Applies the fx_patterns rewrites to a torch.fx GraphModule.

Same surface as the reference optimizer (zenith/optimization/fx_optimizer.py:
43-209): `OptimizationStats`, `FXOptimizer(enable_attention,
enable_activation, enable_normalization, verbose)`, `.optimize(gm,
example_inputs)`, `.get_stats()`, `optimize_fx_graph(...)`,
`is_fx_available()`.

Differences:
  - patterns run in priority order within each group, so a fused pattern
    (Linear+GELU, Add+LayerNorm) claims its nodes before the single-op
    pattern that would split it;
  - a graph whose example inputs are not CUDA tensors is left untouched
    (the replacements are HIP kernels); `stats.skipped_reason` says why;
  - a failure inside the rewriter is counted and re-raised when
    `strict=True` instead of being swallowed.
"""

from __future__ import annotations

import logging
from dataclasses import dataclass, field
from typing import Any, Optional

import torch
import torch.fx
from torch.fx import subgraph_rewriter

from . import fx_patterns as P

logger = logging.getLogger("zenith_amd.hooks.fx_optimizer")


@dataclass
class OptimizationStats:
    total_patterns_checked: int = 0
    patterns_matched: int = 0
    patterns_replaced: int = 0
    patterns_failed: int = 0
    passes_applied: list[str] = field(default_factory=list)
    skipped_reason: Optional[str] = None


def _on_gpu(example_inputs) -> bool:
    """True unless some example input is a tensor that is not on a GPU."""
    if not example_inputs:
        return True
    tensors = [t for t in example_inputs if isinstance(t, torch.Tensor)]
    return all(t.is_cuda for t in tensors) if tensors else True


class FXOptimizer:
    def __init__(self, enable_attention: bool = True, enable_activation: bool = True,
                 enable_normalization: bool = True, verbose: bool = False,
                 strict: bool = False, require_gpu_inputs: bool = True):
        self.enable_attention = enable_attention
        self.enable_activation = enable_activation
        self.enable_normalization = enable_normalization
        self.verbose = verbose
        self.strict = strict
        self.require_gpu_inputs = require_gpu_inputs
        self.stats = OptimizationStats()

    def _groups(self):
        groups = []
        if self.enable_attention:
            groups.append(P.get_attention_patterns())
        if self.enable_activation:
            groups.append(P.get_activation_patterns())
        if self.enable_normalization:
            groups.append(P.get_normalization_patterns())
        return groups

    def optimize(self, gm: torch.fx.GraphModule, example_inputs: Optional[list] = None):
        self.stats = OptimizationStats()
        if self.require_gpu_inputs and not _on_gpu(example_inputs):
            self.stats.skipped_reason = "example inputs are not on a GPU"
            return gm
        for group in self._groups():
            for pattern in sorted(group, key=lambda p: -p.priority):
                if pattern.enabled:
                    self._apply_pattern(gm, pattern)
        gm.graph.lint()
        gm.recompile()
        if self.verbose:
            logger.info("FX optimisation: %s", self.stats)
        return gm

    def _apply_pattern(self, gm: torch.fx.GraphModule, pattern: P.FXPattern):
        self.stats.total_patterns_checked += 1
        try:
            replaced = subgraph_rewriter.replace_pattern(gm, pattern.pattern_fn,
                                                         pattern.replacement_fn)
        except Exception:
            self.stats.patterns_failed += 1
            if self.strict:
                raise
            logger.debug("pattern %s failed", pattern.name, exc_info=True)
            return gm
        if replaced:
            self.stats.patterns_matched += 1
            self.stats.patterns_replaced += len(replaced)
            self.stats.passes_applied.append(pattern.name)
            if self.verbose:
                logger.info("pattern %s matched %d times", pattern.name, len(replaced))
        return gm

    def get_stats(self) -> OptimizationStats:
        return self.stats


def optimize_fx_graph(gm: Any, example_inputs: Optional[list] = None, **kwargs) -> Any:
    """One-shot FXOptimizer(**kwargs).optimize(gm, example_inputs)."""
    return FXOptimizer(**kwargs).optimize(gm, example_inputs)


def is_fx_available() -> bool:
    return hasattr(torch, "fx")


def replaced_targets(gm: torch.fx.GraphModule) -> list[str]:
    """Names of the HIP replacement functions a rewritten graph calls."""
    names = {f.__name__ for f in (P.zenith_sdpa_replacement, P.zenith_gelu_replacement,
                                  P.zenith_gelu_erf_replacement, P.zenith_linear_gelu_replacement,
                                  P.zenith_layernorm_replacement,
                                  P.zenith_add_layernorm_replacement)}
    return [n.target.__name__ for n in gm.graph.nodes
            if n.op == "call_function" and getattr(n.target, "__name__", None) in names]

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
    `strict=True` instead of being swallowed;
  - plain Linear layers (`enable_linear`, default on) go to the HIP GEMM;
  - after the subgraph patterns, a structural pass rewrites the forms real
    models and torch.compile graphs contain, which the literal patterns
    cannot match: nn.Linear / nn.LayerNorm / nn.GELU modules, F.layer_norm
    with a constant normalized shape, F.scaled_dot_product_attention
    without dropout or causal flag, unmasked or with a boolean mask. Where
    the graph carries shape metadata, an attention whose head_dim exceeds
    the kernel's 128 is left alone.
"""

from __future__ import annotations

import logging
import operator
from dataclasses import dataclass, field
from typing import Any, Optional

import torch
import torch.fx
import torch.nn.functional as F
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
                 strict: bool = False, require_gpu_inputs: bool = True,
                 enable_linear: bool = True):
        self.enable_attention = enable_attention
        self.enable_activation = enable_activation
        self.enable_normalization = enable_normalization
        self.verbose = verbose
        self.strict = strict
        self.require_gpu_inputs = require_gpu_inputs
        self.enable_linear = enable_linear
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
        self._structural(gm)
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

    # ------------------------------------------------- structural pass ---
    def _structural(self, gm: torch.fx.GraphModule) -> None:
        g = gm.graph
        mods = dict(gm.named_modules())
        count: dict[str, int] = {}

        def bump(name):
            count[name] = count.get(name, 0) + 1

        def replace(node, fn, args):
            with g.inserting_before(node):
                new = g.call_function(fn, tuple(args))
            new.meta.update(node.meta)
            node.replace_all_uses_with(new)
            g.erase_node(node)
            return new

        for node in list(g.nodes):
            if node.graph is not g or node.op not in ("call_function", "call_module"):
                continue
            if self.enable_attention:
                sd = _as_sdpa(node)
                if sd is not None:
                    replace(node, P.hip_attention, sd)
                    bump("structural_sdpa_to_flash")
                    continue
            if self.enable_activation:
                x = _as_gelu(node, mods)
                if x is not None:
                    lin = _as_linear(gm, x[0], mods) if len(x[0].users) == 1 else None
                    if lin is not None and x[1] == "none":
                        src = x[0]
                        replace(node, P.hip_linear_gelu, lin)
                        g.erase_node(src)
                        bump("structural_linear_gelu")
                    else:
                        replace(node, P.hip_gelu_erf if x[1] == "none" else P.hip_gelu_tanh,
                                [x[0]])
                        bump("structural_gelu")
                    continue
            if self.enable_normalization:
                ln = _as_layernorm(gm, node, mods)
                if ln is not None:
                    inp, w, b, eps = ln
                    if (inp.op == "call_function" and inp.target in _ADD and len(inp.users) == 1
                            and len(inp.args) == 2 and not inp.kwargs
                            and all(isinstance(a, torch.fx.Node) for a in inp.args)
                            and _same_shape(*inp.args)):
                        a0, a1 = inp.args
                        replace(node, P.hip_add_layernorm_eps, [a0, a1, w, b, eps])
                        g.erase_node(inp)
                        bump("structural_add_layernorm")
                    else:
                        replace(node, P.hip_layernorm, [inp, w, b, eps])
                        bump("structural_layernorm")
                    continue
            if self.enable_linear and not _feeds_gelu(node, mods):
                lin = _as_linear(gm, node, mods)
                if lin is not None:
                    replace(node, P.hip_linear, lin)
                    bump("structural_linear")
                    continue
        for name, n in count.items():
            self.stats.patterns_matched += 1
            self.stats.patterns_replaced += n
            self.stats.passes_applied.append(name)
        g.eliminate_dead_code()


def optimize_fx_graph(gm: Any, example_inputs: Optional[list] = None, **kwargs) -> Any:
    """One-shot FXOptimizer(**kwargs).optimize(gm, example_inputs)."""
    return FXOptimizer(**kwargs).optimize(gm, example_inputs)


def is_fx_available() -> bool:
    return hasattr(torch, "fx")


def replaced_targets(gm: torch.fx.GraphModule) -> list[str]:
    """Names of the HIP leaf functions a rewritten graph calls."""
    leaves = {f.__name__ for f in (P.hip_flash_attention, P.hip_gelu_tanh, P.hip_gelu_erf,
                                   P.hip_linear_gelu, P.hip_layernorm, P.hip_add_layernorm,
                                   P.hip_add_layernorm_eps, P.hip_attention, P.hip_linear)}
    return [n.target.__name__ for n in gm.graph.nodes
            if n.op == "call_function" and getattr(n.target, "__name__", None) in leaves]


# ------------------------------------------------ structural matchers ----
_LINEAR = {F.linear, torch._C._nn.linear}
_GELU = {F.gelu, torch._C._nn.gelu}
_LAYERNORM = {F.layer_norm, torch.layer_norm}
_ADD = {operator.add, operator.iadd, torch.add}
_MAX_HEAD_DIM = 128  # the kernel's limit (the reference's HEAD_DIM_MAX)


def _arg(node, i, name, default=None):
    if len(node.args) > i:
        return node.args[i]
    return node.kwargs.get(name, default)


def _param(gm, node, mod_name, attr):
    """get_attr node for a submodule parameter, inserted before `node`."""
    if getattr(gm.get_submodule(mod_name), attr) is None:
        return None
    with gm.graph.inserting_before(node):
        return gm.graph.get_attr(f"{mod_name}.{attr}")


def _as_linear(gm, node, mods):
    """(x, W[N,K], b) of F.linear(x, W, b) or an nn.Linear call, else None."""
    if node.op == "call_function" and node.target in _LINEAR:
        return [_arg(node, 0, "input"), _arg(node, 1, "weight"), _arg(node, 2, "bias")]
    if node.op == "call_module" and isinstance(mods.get(node.target), torch.nn.Linear):
        return [node.args[0], _param(gm, node, node.target, "weight"),
                _param(gm, node, node.target, "bias")]
    return None


def _as_gelu(node, mods):
    """(input, approximate) of a GELU call, else None."""
    if node.op == "call_function" and node.target in _GELU:
        return node.args[0], _arg(node, 1, "approximate", "none")
    if node.op == "call_module" and isinstance(mods.get(node.target), torch.nn.GELU):
        return node.args[0], mods[node.target].approximate
    return None


def _as_layernorm(gm, node, mods):
    """(input, gamma, beta, eps) of a LayerNorm over the last dimension with
    an affine transform, else None."""
    if node.op == "call_function" and node.target in _LAYERNORM:
        shape = _arg(node, 1, "normalized_shape")
        w, b = _arg(node, 2, "weight"), _arg(node, 3, "bias")
        if not isinstance(shape, (tuple, list)) or len(shape) != 1 or w is None or b is None:
            return None
        return node.args[0], w, b, float(_arg(node, 4, "eps", 1e-5))
    if node.op == "call_module" and isinstance(mods.get(node.target), torch.nn.LayerNorm):
        m = mods[node.target]
        if len(m.normalized_shape) != 1 or m.weight is None or m.bias is None:
            return None
        return (node.args[0], _param(gm, node, node.target, "weight"),
                _param(gm, node, node.target, "bias"), float(m.eps))
    return None


def _meta_last_dim(node):
    for key in ("val", "example_value", "tensor_meta"):
        v = node.meta.get(key) if isinstance(node, torch.fx.Node) else None
        shape = getattr(v, "shape", None)
        if shape is not None and len(shape):
            try:
                return int(shape[-1])
            except (TypeError, ValueError):
                return None
    return None


def _meta_shape(node):
    for key in ("val", "example_value", "tensor_meta"):
        v = node.meta.get(key) if isinstance(node, torch.fx.Node) else None
        shape = getattr(v, "shape", None)
        if shape is not None:
            return tuple(shape)
    return None


def _same_shape(a, b) -> bool:
    """False when the graph's shape metadata shows a and b differ (an Add
    that broadcasts, such as BERT's embeddings + [1, S, H] position term,
    stays a torch add in front of the HIP LayerNorm); True when they agree
    or the graph carries no metadata (the fused leaf broadcasts itself)."""
    sa, sb = _meta_shape(a), _meta_shape(b)
    return sa is None or sb is None or sa == sb


def _meta_dtype(node):
    for key in ("val", "example_value", "tensor_meta"):
        v = node.meta.get(key) if isinstance(node, torch.fx.Node) else None
        dt = getattr(v, "dtype", None)
        if dt is not None:
            return dt
    return None


def _as_sdpa(node):
    """(q, k, v, scale, attn_mask) of a non-causal, dropout-free
    scaled_dot_product_attention whose mask is absent or boolean (True =
    attend; known from the graph's shape metadata, as torch.compile graphs
    carry it: HF BERT's SDPA path passes a boolean [B, 1, Sq, Sk] padding
    mask), else None. Additive float masks, and masks of unknown dtype, stay
    with torch."""
    if node.op != "call_function" or node.target is not F.scaled_dot_product_attention:
        return None
    q, k, v = node.args[:3]
    mask = _arg(node, 3, "attn_mask")
    if _arg(node, 5, "is_causal", False):
        return None
    if mask is not None and (not isinstance(mask, torch.fx.Node) or _meta_dtype(mask) != torch.bool):
        return None
    if float(_arg(node, 4, "dropout_p", 0.0) or 0.0) != 0.0 or _arg(node, 7, "enable_gqa", False):
        return None
    d = _meta_last_dim(q)
    if d is not None and d > _MAX_HEAD_DIM:
        return None
    return [q, k, v, _arg(node, 6, "scale"), mask]


def _feeds_gelu(node, mods) -> bool:
    """A Linear whose only user is a GELU is left for the Linear+GELU fusion."""
    return len(node.users) == 1 and _as_gelu(next(iter(node.users)), mods) is not None

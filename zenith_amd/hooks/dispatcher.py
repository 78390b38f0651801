"""Routes graph nodes (op_type, inputs, outputs, attributes) to the HIP
kernels through the registry.

Same surface as the reference dispatcher (zenith/runtime/dispatcher.py:
24-396): `DispatchTarget`, `KernelDispatcher(registry, precision, device)`
with `OP_TYPE_MAP`, `dispatch(node, context, weights)`,
`get_dispatch_stats()`, `reset_stats()`, and the exceptions
`UnsupportedOperationError` / `KernelExecutionError`. The argument
marshalling is per op type as in `_call_kernel` (dispatcher.py:235-315),
with these corrections:

  - Linear is called as fn(x, W[N,K], b); ONNX `Gemm` honours transB and
    `MatMul` with a weight treats it as B[K,N] (both become Linear);
    `MatMul` of two activations stays a plain A[M,K] . B[K,N] product.
    (The reference normalised MatMul/Gemm to Linear and passed three
    arguments to the two-argument matmul, dispatcher.py:251-254.)
  - the fused op types produced by the graph passes dispatch to fused
    kernels instead of raising UnsupportedOperationError.
  - `TorchExported` nodes (whole-model fallback, dispatcher.py:347-389) are
    not supported: this dispatcher only runs HIP kernels.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Optional

from .kernel_registry import KernelRegistry, KernelSpec, Precision, get_registry


class UnsupportedOperationError(Exception):
    pass


class KernelExecutionError(Exception):
    pass


@dataclass
class Node:
    """Minimal graph node: what the dispatcher reads from a GraphIR node."""

    op_type: str
    inputs: list
    outputs: list
    attributes: dict = field(default_factory=dict)
    name: str = ""


class ExecutionContext:
    """Name -> tensor store of one graph execution."""

    def __init__(self, tensors: Optional[dict] = None):
        self._t = dict(tensors or {})
        self._meta: dict = {}

    def has_tensor(self, name: str) -> bool:
        return name in self._t

    def get_tensor(self, name: str):
        return self._t[name]

    def set_tensor(self, name: str, value) -> None:
        self._t[name] = value

    def get_metadata(self, key: str, default=None):
        return self._meta.get(key, default)

    def set_metadata(self, key: str, value) -> None:
        self._meta[key] = value


@dataclass
class DispatchTarget:
    kernel_spec: KernelSpec
    input_names: list
    output_names: list
    weights: Optional[dict] = None
    attributes: Optional[dict] = None


def _name(t) -> str:
    if isinstance(t, str):
        return t
    return getattr(t, "name", str(t))


class KernelDispatcher:
    OP_TYPE_MAP = {
        "Gemm": "Linear",
        "LayerNormalization": "LayerNorm",
        "Relu": "ReLU",
        "Gelu": "GELU",
        "MultiHeadAttention": "Attention",
        "AddLayerNorm": "FusedAddLayerNorm",
        "Add+LayerNorm": "FusedAddLayerNorm",
        "BiasGeLU": "FusedBiasGeLU",
        "Bias+GELU": "FusedBiasGeLU",
        "FusedLinearGelu": "LinearGelu",
        "FusedLayerNormAdd": "LayerNormAdd",
        "flash_attention": "FlashAttention",
    }

    def __init__(self, registry: Optional[KernelRegistry] = None,
                 precision: Precision = Precision.FP32, device: str = "cuda"):
        self.registry = registry or get_registry()
        self.precision = precision
        self.device = device
        self._dispatch_count = 0
        self._kernel_usage: dict[str, int] = {}

    def _normalize_op_type(self, op_type: str) -> str:
        return self.OP_TYPE_MAP.get(op_type, op_type)

    def dispatch(self, node: Any, context: ExecutionContext, weights: Optional[dict] = None):
        raw_op = getattr(node, "op_type", str(node))
        op = self._normalize_op_type(raw_op)
        names = [_name(i) for i in getattr(node, "inputs", [])]
        inputs = [context.get_tensor(n) for n in names if context.has_tensor(n)]
        shapes = [tuple(getattr(t, "shape", ())) for t in inputs]
        lookup = "Linear" if op == "MatMul" and weights else op
        kernel = self.registry.get_kernel(lookup, self.precision, shapes)
        if kernel is None:
            raise UnsupportedOperationError(
                f"No kernel found for operation '{raw_op}' with precision "
                f"{self.precision.value}. Supported operations: {self.registry.list_supported_ops()}")
        attrs = dict(getattr(node, "attributes", None) or {})
        try:
            out = self._call_kernel(kernel, op, raw_op, inputs, weights or {}, attrs)
        except (UnsupportedOperationError, KernelExecutionError):
            raise
        except Exception as e:  # noqa: BLE001 - re-raised with context
            raise KernelExecutionError(
                f"Kernel {kernel.name} failed: {e}. Inputs: {shapes}") from e
        outs = [_name(o) for o in getattr(node, "outputs", [])]
        if outs:
            if isinstance(out, tuple):
                for n, t in zip(outs, out):
                    context.set_tensor(n, t)
            else:
                context.set_tensor(outs[0], out)
        self._dispatch_count += 1
        self._kernel_usage[kernel.name] = self._kernel_usage.get(kernel.name, 0) + 1
        return out

    @staticmethod
    def _w(weights: dict, *keys):
        for k in keys:
            if k in weights:
                return weights[k]
        return None

    def _call_kernel(self, kernel: KernelSpec, op: str, raw_op: str, inputs: list,
                     weights: dict, attrs: dict):
        fn = kernel.kernel_fn
        if fn is None:
            raise RuntimeError(f"Kernel {kernel.name} has no implementation")
        w = self._w
        eps = attrs.get("epsilon", attrs.get("eps", 1e-5))
        if op in ("Linear", "MatMul"):
            W = w(weights, "weight", "W", "B")
            b = w(weights, "bias", "b", "C")
            if W is None:
                if op == "MatMul" and len(inputs) >= 2:
                    return fn(inputs[0], inputs[1])
                raise KernelExecutionError(f"{raw_op}: no weight given")
            if raw_op == "MatMul" or (raw_op == "Gemm" and not attrs.get("transB", 0)):
                W = W.t()  # B[K, N] -> W[N, K]
            if self.precision == Precision.INT8:
                return fn(inputs[0], W, attrs["s_x"], w(weights, "s_w"), b)
            return fn(inputs[0], W, b)
        if op == "LinearGelu":
            return fn(inputs[0], w(weights, "weight", "W"), w(weights, "bias", "b"),
                      attrs.get("approximate", "none"))
        if op == "LayerNorm":
            return fn(inputs[0], w(weights, "weight", "gamma", "scale"),
                      w(weights, "bias", "beta", "B"), eps)
        if op == "FusedAddLayerNorm":
            return fn(inputs[0], inputs[1], w(weights, "weight", "gamma"),
                      w(weights, "bias", "beta"), eps)
        if op == "LayerNormAdd":
            # LayerNormalization(x, scale, B) -> Add(., residual): either the
            # four node inputs in that order, or (x, residual) with the affine
            # parameters as weights
            if len(inputs) >= 4:
                return fn(inputs[0], inputs[3], inputs[1], inputs[2], eps)
            return fn(inputs[0], inputs[1], w(weights, "weight", "gamma", "scale"),
                      w(weights, "bias", "beta", "B"), eps)
        if op == "GELU":
            return fn(inputs[0], attrs.get("approximate", "tanh"))
        if op == "FusedBiasGeLU":
            bias = inputs[1] if len(inputs) > 1 else w(weights, "bias")
            return fn(inputs[0], bias, attrs.get("approximate", "tanh"))
        if op == "ReLU":
            return fn(inputs[0])
        if op in ("Attention", "FlashAttention"):
            if len(inputs) < 3:
                raise KernelExecutionError(f"{raw_op}: expects q, k, v inputs")
            lens = inputs[3] if len(inputs) > 3 else attrs.get("key_padding_lengths")
            return fn(inputs[0], inputs[1], inputs[2], key_padding_lengths=lens,
                      scale=attrs.get("scale"))
        if op == "QKVProjection":
            return fn(inputs[0], w(weights, "Wq"), w(weights, "bq"), w(weights, "Wk"),
                      w(weights, "bk"), w(weights, "Wv"), w(weights, "bv"))
        if op == "FusedAttentionEpilogue":
            return fn(inputs[0], inputs[1], w(weights, "weight", "Wo"), w(weights, "bias", "bo"),
                      w(weights, "gamma"), w(weights, "beta"), attrs.get("epsilon", 1e-12))
        if op == "FusedFFN":
            return fn(inputs[0], w(weights, "Wi"), w(weights, "bi"), w(weights, "Wo2"),
                      w(weights, "bo2"), w(weights, "gamma"), w(weights, "beta"),
                      attrs.get("epsilon", 1e-12))
        return fn(*inputs, *weights.values())

    def get_dispatch_stats(self) -> dict:
        return {"total_dispatches": self._dispatch_count,
                "kernel_usage": dict(self._kernel_usage),
                "precision": self.precision.value, "device": self.device}

    def reset_stats(self) -> None:
        self._dispatch_count = 0
        self._kernel_usage.clear()

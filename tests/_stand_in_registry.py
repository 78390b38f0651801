"""Stand-in for the reference's kernel registry module
(zenith/runtime/kernel_registry.py:22-153), for CPU tests of the
reference-side binding. It defines its OWN Precision enum and KernelSpec
class, as the reference module does, and selects kernels the way the
reference's get_kernel does: keep the specs whose `precision == precision`
(enum identity), drop those whose constraints fail, return the highest
priority, and retry with FP32 when nothing is left."""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum
from typing import Callable, Optional


class Precision(Enum):
    FP32 = "fp32"
    FP16 = "fp16"
    BF16 = "bf16"
    INT8 = "int8"


@dataclass
class KernelSpec:
    name: str
    op_types: list
    precision: Precision
    kernel_fn: Optional[Callable] = None
    input_constraints: dict = field(default_factory=dict)
    priority: int = 0
    estimated_flops: Optional[Callable] = None
    requires_gpu: bool = True

    def check_constraints(self, input_shapes) -> bool:
        return True


class KernelRegistry:
    def __init__(self):
        self._kernels: dict = {}

    def register(self, spec: KernelSpec) -> None:
        for op in spec.op_types:
            self._kernels.setdefault(op, []).append(spec)

    def get_kernel(self, op_type, precision, input_shapes=None):
        found = self._kernels.get(op_type, [])
        if not found:
            return None
        found = [k for k in found if k.precision == precision]
        if input_shapes:
            found = [k for k in found if k.check_constraints(input_shapes)]
        if not found:
            return self.get_kernel(op_type, Precision.FP32, input_shapes) \
                if precision != Precision.FP32 else None
        return sorted(found, key=lambda k: -k.priority)[0]

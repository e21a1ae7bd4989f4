"""LerpTensorFwdOp: y = torch.lerp(input, end, weight) with a weight tensor.

Reference: examples/TileOPs/tileops/ops/elementwise/lerp_tensor.py:35-165
(constructor ``(*, input: shape, end: shape, weight: shape, dtype)``, float
dtypes for all three operands, the rejection message "LerpTensorFwdOp does
not support dtype ...", three-way broadcast, constructor-named attributes;
roofline flops ``3 * N``, bytes ``4 * N * elem_bytes``).  Broadcast operands
are read in place by the kernel rather than expanded into copies.
"""

from __future__ import annotations

from math import prod
from typing import Dict, Optional

import torch

from tileops.device import get_device_backend
from tileops.kernels.elementwise.lerp_tensor import LerpTensorFwdKernel
from tileops.kernels.kernel_base import Kernel
from tileops.ops.op_base import Op

__all__ = ["LerpTensorFwdOp"]


class LerpTensorFwdOp(Op):
    """Tensor-weight lerp: ``input + weight * (end - input)``, all broadcast.

    Args:
        input: Shape of the start tensor.
        end: Shape of the end tensor.
        weight: Shape of the per-element weight tensor.
        dtype: float16, bfloat16 or float32 (all three operands).
        kernel_map: Optional kernel dispatch override.
    """

    _op_name = "lerp_tensor"
    _SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

    def __init__(self, *, input: tuple, end: tuple, weight: tuple, dtype: torch.dtype,
                 kernel_map: Optional[Dict[str, Kernel]] = None):
        if dtype not in self._SUPPORTED_DTYPES:
            names = ", ".join(str(dt) for dt in self._SUPPORTED_DTYPES)
            raise ValueError(
                f"LerpTensorFwdOp does not support dtype {dtype}. Supported: [{names}]")
        self.input = tuple(input)
        self.end = tuple(end)
        self.weight = tuple(weight)
        self.input_shape = self.input
        self.end_shape = self.end
        self.weight_shape = self.weight
        self.dtype = dtype
        self.output_dtype = dtype
        self.out_shape = tuple(
            torch.broadcast_shapes(self.input_shape, self.end_shape, self.weight_shape))
        self.N_total = prod(self.out_shape) if self.out_shape else 1
        self.dispatch_kernel(kernel_map)
        self.kernel = self.kernel_map[self._op_name](self.N_total, dtype)

    @property
    def default_kernel_map(self) -> Dict[str, Kernel]:
        return {self._op_name: LerpTensorFwdKernel}

    def forward(self, input: torch.Tensor, end: torch.Tensor,
                weight: torch.Tensor) -> torch.Tensor:
        backend = get_device_backend()
        if not (backend.is_device_tensor(input) and backend.is_device_tensor(end)
                and backend.is_device_tensor(weight)):
            raise ValueError(f"Inputs must be {backend.name} tensors")
        for name, t, expected in (("input", input, self.input_shape),
                                  ("end", end, self.end_shape),
                                  ("weight", weight, self.weight_shape)):
            if t.dtype != self.dtype:
                raise ValueError(f"Expected {name}.dtype {self.dtype}, got {t.dtype}")
            if tuple(t.shape) != expected:
                raise ValueError(f"Expected {name}.shape {expected}, got {tuple(t.shape)}")
        return self.kernel(input, end, weight)

    def eval_roofline(self) -> tuple[int, int]:
        n_total = int(self.N_total)
        return 3 * n_total, 4 * n_total * self.dtype.itemsize

"""LerpFwdOp: y = torch.lerp(input, end, weight) with a scalar weight.

Reference: examples/TileOPs/tileops/ops/elementwise/lerp_scalar.py:38-157
(constructor ``(*, input: shape, end: shape, dtype, weight=0.5)``, float
dtypes, the rejection message "LerpFwdOp does not support dtype ...",
``out_shape = broadcast_shapes(input, end)``, constructor-named attributes;
roofline flops ``3 * N``, bytes ``4 * N * elem_bytes`` with N the broadcast
element count).  The reference expanded both operands to the output shape
and flattened them; here the kernel reads broadcast operands in place.
"""

from __future__ import annotations

from math import prod
from typing import Dict, Optional

import torch

from tileops.device import get_device_backend
from tileops.kernels.elementwise.lerp_scalar import LerpScalarFwdKernel
from tileops.kernels.kernel_base import Kernel
from tileops.ops.op_base import Op

__all__ = ["LerpFwdOp"]


class LerpFwdOp(Op):
    """Scalar-weight lerp with broadcasting: ``input + weight * (end - input)``.

    Args:
        input: Shape of the start tensor.
        end: Shape of the end tensor (broadcasts against ``input``).
        dtype: float16, bfloat16 or float32 (both operands).
        weight: Interpolation weight (default 0.5), fixed per Op instance.
        kernel_map: Optional kernel dispatch override.
    """

    _op_name = "lerp_scalar"
    _SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

    def __init__(self, *, input: tuple, end: tuple, dtype: torch.dtype, weight: float = 0.5,
                 kernel_map: Optional[Dict[str, Kernel]] = None):
        if dtype not in self._SUPPORTED_DTYPES:
            names = ", ".join(str(dt) for dt in self._SUPPORTED_DTYPES)
            raise ValueError(f"LerpFwdOp does not support dtype {dtype}. Supported: [{names}]")
        self.input = tuple(input)
        self.end = tuple(end)
        self.input_shape = self.input
        self.end_shape = self.end
        self.dtype = dtype
        self.weight = weight
        self.output_dtype = dtype
        self.out_shape = tuple(torch.broadcast_shapes(self.input_shape, self.end_shape))
        self.N_total = prod(self.out_shape) if self.out_shape else 1
        self.dispatch_kernel(kernel_map)
        self.kernel = self.kernel_map[self._op_name](self.N_total, dtype, self.weight)

    @property
    def default_kernel_map(self) -> Dict[str, Kernel]:
        return {self._op_name: LerpScalarFwdKernel}

    def forward(self, input: torch.Tensor, end: torch.Tensor) -> torch.Tensor:
        backend = get_device_backend()
        if not (backend.is_device_tensor(input) and backend.is_device_tensor(end)):
            raise ValueError(f"Inputs must be {backend.name} tensors")
        for name, t, expected in (("input", input, self.input_shape),
                                  ("end", end, self.end_shape)):
            if t.dtype != self.dtype:
                raise ValueError(f"Expected {name}.dtype {self.dtype}, got {t.dtype}")
            if tuple(t.shape) != expected:
                raise ValueError(f"Expected {name}.shape {expected}, got {tuple(t.shape)}")
        return self.kernel(input, end)

    def eval_roofline(self) -> tuple[int, int]:
        n_total = int(self.N_total)
        return 3 * n_total, 4 * n_total * self.dtype.itemsize
